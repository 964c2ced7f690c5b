// Device helpers shared by the int8 and int4 decode kernels: lane-group
// reductions, the hi/lo pair swap, vector loads of a Q chunk, RoPE of one
// element, and the (sequence, split) mapping of a decode workgroup.
//
// Wave layout used by both kernels: lane = r + 16 g (r = lane & 15 is the
// MFMA row/column index, g = lane >> 4 the lane group, i.e. the page of the
// current 64-token tile).
#pragma once

#include "sai_internal.h"

namespace sai {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kMaxSplitPages = 1024;  // split_tokens <= 16384 (page ids staged in LDS)

// RoPE of one element; `first` = this element is x0 of its pair. Both
// products are rounded on their own and the select picks the sign of the
// second, so x0: c*x0 - s*x1 and x1: s*x0 + c*x1 (== c*x1 + s*x0) without a
// branch per lane.
__device__ __forceinline__ float rope_elem(float c, float s, float own, float partner,
                                           bool first) {
#pragma clang fp contract(off)
  const float a = c * own;
  const float b = s * partner;
  return a + (first ? -b : b);
}

__device__ __forceinline__ int pack4(int a, int b, int c, int d) {
  return (a & 0xFF) | ((b & 0xFF) << 8) | ((c & 0xFF) << 16) | ((int)((unsigned)d << 24));
}

// exchange with the neighbouring lane: quad_perm(1,0,3,2)
__device__ __forceinline__ int swap_pair(int v) {
  return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);
}

// max / sum over the four lane groups (lanes r, r+16, r+32, r+48)
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

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <int K>
__device__ __forceinline__ float comp4(const float4& v) {
  if constexpr (K == 0) return v.x;
  else if constexpr (K == 1) return v.y;
  else if constexpr (K == 2) return v.z;
  else return v.w;
}

// Element I of 16 table entries loaded as four float4 q[0..3] from the run's
// start: split-half pairs take entry I, interleaved pairs entry I / 2. Both
// candidates are constant components of SSA values, so the select stays a
// v_cndmask (a select between two elements of one local array is turned into
// dynamic register indexing, which waits for the loads at once).
template <int I>
__device__ __forceinline__ float rope_pick(const float4 (&q)[4], bool interleaved) {
  const float split_half = comp4<I & 3>(q[I >> 2]);
  const float inter = comp4<(I >> 1) & 3>(q[I >> 3]);
  return interleaved ? inter : split_half;
}

template <int I>
__device__ __forceinline__ void rope_pick_all(const float4 (&qc)[4], const float4 (&qs)[4],
                                              bool interleaved, float (&c)[16], float (&s)[16]) {
  c[I] = rope_pick<I>(qc, interleaved);
  s[I] = rope_pick<I>(qs, interleaved);
  if constexpr (I + 1 < 16) rope_pick_all<I + 1>(qc, qs, interleaved, c, s);
}

// The cos / sin table entries of the 16 dims [c0, c0 + 16) of a query row at
// one position (cr, sr: that position's table rows of head_dim / 2 entries,
// 16-byte aligned): split-half pairs use entries c0 mod (D/2) + i,
// interleaved pairs entry (c0 + i) / 2. rope_load16 issues four 16-byte loads
// per table whatever the pairing (interleaved needs the first two; the other
// two repeat them, since base + 16 may pass the row end), 8 loads instead of
// 32; rope_pick_all turns them into per-dim values where they are used, so
// that nothing waits for the loads before then.
template <int D>
__device__ __forceinline__ void rope_load16(const float* cr, const float* sr, int c0,
                                            int interleaved, float4 (&qc)[4], float4 (&qs)[4]) {
  constexpr int HALF = D / 2;
  const bool il = interleaved != 0;
  const int base = il ? (c0 >> 1) : (c0 < HALF ? c0 : c0 - HALF);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int off = base + 4 * (il ? (j & 1) : j);
    qc[j] = *(const float4*)(cr + off);
    qs[j] = *(const float4*)(sr + off);
  }
}

// Split partials handed between workgroups of one launch. The workgroups of
// a (sequence, kv head) run on different XCDs, whose L2 caches are not kept
// coherent with each other for ordinary stores. An agent-scope atomic store or
// load is coherent across them by itself (gfx950 emits global_store /
// global_load with sc1), so the handoff needs no L2 writeback or invalidate:
// the writer stores its partial this way, waits for the stores to complete
// (partials_complete), and only then takes a ticket from the counter; the
// workgroup with the last ticket loads the other partials this way.
__device__ __forceinline__ void store_partial(float* a, float v) {
  __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_partial(const float* a) {
  return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Every vector memory access of this wave issued so far has completed (on
// gfx9 vmcnt counts stores until they are acknowledged); also a compiler
// barrier, so no store is moved past it.
__device__ __forceinline__ void partials_complete() {
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
}
// One ticket of the split counter of a (sequence, kv head); true for the
// workgroup that takes the last one, which then resets the counter for the
// next launch. Call after partials_complete() and a workgroup barrier.
__device__ __forceinline__ bool last_ticket(int* counter, int nsplit) {
  return __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
         nsplit - 1;
}
__device__ __forceinline__ void reset_ticket(int* counter) {
  __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Online merge of the splits' (m, l, o) entries for one (head, dim) into
// (M, Ls, O), C splits per round trip, in split order, skipping split `own`
// (-1: none) and splits with no visible key; `ph` points at split 0's (m, l,
// o[...]) block of this head, `stride` floats apart per split, `d` the dim.
template <int C>
__device__ __forceinline__ void merge_partials(const float* ph, size_t stride, int d, int nsplit,
                                               int own, float& M, float& Ls, float& O) {
  for (int s0 = 0; s0 < nsplit; s0 += C) {
    float m[C], l[C], o[C];
#pragma unroll
    for (int i = 0; i < C; ++i) {
      const int s = min(s0 + i, nsplit - 1);
      const float* ps = ph + (size_t)s * stride;
      m[i] = load_partial(ps);
      l[i] = load_partial(ps + 1);
      o[i] = load_partial(ps + 2 + d);
    }
#pragma unroll
    for (int i = 0; i < C; ++i) {
      const int s = s0 + i;
      if (s >= nsplit || s == own || m[i] == -INFINITY) continue;
      const float mn = fmaxf(M, m[i]);
      const float fa = M == -INFINITY ? 0.0f : fast_exp2(M - mn);
      const float fb = fast_exp2(m[i] - mn);
      Ls = Ls * fa + l[i] * fb;
      O = O * fa + o[i] * fb;
      M = mn;
    }
  }
}

// merge_partials with the batch width picked from the split count: all of a
// (head, dim) entry's splits in one round trip up to 32 splits (each round
// trip to partials written on other XCDs costs a full memory latency).
__device__ __forceinline__ void merge_all_splits(const float* ph, size_t stride, int d,
                                                 int nsplit, float& M, float& Ls, float& O) {
  if (nsplit <= 2)
    merge_partials<2>(ph, stride, d, nsplit, -1, M, Ls, O);
  else if (nsplit <= 4)
    merge_partials<4>(ph, stride, d, nsplit, -1, M, Ls, O);
  else if (nsplit <= 8)
    merge_partials<8>(ph, stride, d, nsplit, -1, M, Ls, O);
  else if (nsplit <= 16)
    merge_partials<16>(ph, stride, d, nsplit, -1, M, Ls, O);
  else
    merge_partials<32>(ph, stride, d, nsplit, -1, M, Ls, O);
}

// 16 consecutive elements (f32 or bf16) starting at element `off`; the
// offset is a multiple of 16 and the row 32-byte aligned.
__device__ __forceinline__ void load16(const void* base, size_t off, int dtype, float (&x)[16]) {
  if (dtype == kDtypeBf16) {
    const uint4* p = (const uint4*)((const uint16_t*)base + off);
    const uint4 a = p[0], b = p[1];
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x[2 * i] = __uint_as_float(w[i] << 16);
      x[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  } else {
    const float4* p = (const float4*)((const float*)base + off);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 v = p[i];
      x[4 * i] = v.x, x[4 * i + 1] = v.y, x[4 * i + 2] = v.z, x[4 * i + 3] = v.w;
    }
  }
}

// (sequence, split) of a decode workgroup and its split's length in 64-token
// tiles. Uniform split count: direct mapping, splits of split_tokens.
// Ragged: a prefix scan over the per-sequence split counts of seq_lens[b] +
// pending tokens (in p.order when given), and a sequence's streamed tiles
// dealt evenly to its splits (ceil(T / nsplit) each, the last split taking
// the rest, never none), so no split is a short remainder. Returns b = -1
// past the last work item.
__device__ __forceinline__ void decode_work_item(const DecodeParams& p, int work, int lane, int& b,
                                                 int& split, int& nsplit, int& split_base,
                                                 int& tps) {
  b = -1;
  split = nsplit = split_base = 0;
  tps = p.split_tokens / 64;
  if (p.uniform_nsplit > 0) {
    nsplit = p.uniform_nsplit;
    b = work / nsplit;
    split = work - b * nsplit;
    split_base = b * nsplit;
    return;
  }
  int base = 0;
  for (int c0 = 0; c0 < p.batch; c0 += 64) {
    const int bi = c0 + lane;
    const int sb = bi < p.batch ? (p.ordered ? (int)p.order[bi] : bi) : 0;
    const int Lb = bi < p.batch ? p.seq_lens[sb] + p.pending : 0;
    const int span = Lb - window_origin(Lb, p.window);
    const int n = (span + p.split_tokens - 1) / p.split_tokens;
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
      b = __shfl(sb, first, 64);
      split_base = base + __shfl(incl - n, first, 64);
      nsplit = __shfl(n, first, 64);
      const int tiles = (__shfl(span, first, 64) + 63) / 64;
      tps = (tiles + nsplit - 1) / nsplit;
      split = work - split_base;
      return;
    }
    base += total;
  }
}

// The length of sequence b (seq_lens[b] + pending) and the split's page ids,
// staged into sm_pg (page slot i of the split = sm_pg[i]). The length is a
// scalar load (b is uniform), so it waits on its own counter; without a
// window the split's first page does not depend on it, and the page-id loads
// go out beside it instead of after it: one memory round trip less before the
// first tile. With a window the split starts at the tile holding the first
// visible key, which needs the length first. NT = threads of the workgroup.
template <int NT>
__device__ __forceinline__ void stage_split_pages(const DecodeParams& p, int b, int split, int tps,
                                                  int* sm_pg, int& L, int& k_lo,
                                                  int& first_page) {
  b = __builtin_amdgcn_readfirstlane(b);
  const int32_t* pt = p.page_table + (size_t)b * p.max_pages;
  const int split_pages = tps * (64 / kPageTokens);
  const int len = p.seq_lens[b];
  if (p.window <= 0) {
    first_page = split * split_pages;
    for (int i = threadIdx.x; i < split_pages; i += NT)
      sm_pg[i] = pt[min(first_page + i, p.max_pages - 1)];
    L = len + p.pending;
    k_lo = 0;
  } else {
    L = len + p.pending;
    k_lo = window_first_key(L, p.window);
    first_page = (k_lo / 64) * 64 / kPageTokens + split * split_pages;
    for (int i = threadIdx.x; i < split_pages; i += NT)
      sm_pg[i] = pt[min(first_page + i, p.max_pages - 1)];
  }
}

}  // namespace sai
