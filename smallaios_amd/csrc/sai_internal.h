// Internal definitions shared by the gfx950 kernels and the C ABI.
//
// Paged cache layout (one pool per layer, page p, kv head h), kv-head major so
// that the pages of one sequence and head (identity or clustered page tables)
// form one contiguous stream for the decode workgroup that reads them:
//   block(p, h) = pool + (h * num_pages + p) * block_bytes
//
// INT8 block, D = stored_head_dim(head_dim) (below), 16 tokens:
//   [0,        16*D)        K codes, row-major [slot][D]        (int8)
//   [16*D,     32*D)        V codes, transposed [D][slot]       (int8)
//   [32*D,     32*D+64)     K scales [slot]                     (f32)
//   [32*D+64,  32*D+128)    V scales [slot]                     (f32)
//   block_bytes = 32*D + 128
// INT4 block (G = D/32 groups):
//   [0,      8*D)           K codes [slot][D/2], LSB-first along D
//   [8*D,    16*D)          V codes [D][8], LSB-first along slots
//   [16*D,   16*D+64*G)     K (scale, zero) binary16 [slot][G][2]
//   [.. ,    16*D+128*G)    V (scale, zero) binary16 [slot][G][2]
//   block_bytes = 16*D + 128*G = 20*D
//
// K is stored token-major so that a decode lane's 16-byte load is 16
// consecutive head_dim codes of one token (the k operand of the QK MFMA);
// V is stored dim-major so that a lane's 16-byte load is 16 consecutive
// tokens of one dim (the k operand of the PV MFMA).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sai {

constexpr int kPageTokens = 16;
constexpr int kQuantInt8 = 1;
constexpr int kQuantInt4 = 2;
constexpr int kDtypeF32 = 1;
constexpr int kDtypeF16 = 10;
constexpr int kDtypeBf16 = 16;

// Stored width of a head's rows in the cache and in the kernels' tiles.
// head_dim 168 (Gemma 4 31B) is stored as 192: each 84-dim half of the
// split-half RoPE pairing gets 12 zero dims after it, so the kernels keep
// whole 16-dim chunks, the pair (i, i + 84) sits at (i, i + 96), interleaved
// pairs stay adjacent, and the zeros change neither a row's int8 scale nor
// any dot product. Every other head_dim is stored as it is.
__host__ __device__ constexpr int stored_head_dim(int head_dim) {
  return head_dim == 168 ? 192 : head_dim;
}
// The head_dim a stored width D serves.
template <int D>
constexpr int kLogicalDim = D == 192 ? 168 : D;
// Dim of the caller's row held by stored dim e of a D-wide row; -1 for a
// padding dim.
template <int D>
__host__ __device__ constexpr int logical_dim(int e) {
  constexpr int DL = kLogicalDim<D>;
  if constexpr (DL == D) {
    return e;
  } else {
    const int h = e >= D / 2 ? 1 : 0;
    const int i = e - h * (D / 2);
    return i < DL / 2 ? i + h * (DL / 2) : -1;
  }
}

__host__ __device__ constexpr size_t block_bytes_int8(int d) { return (size_t)32 * d + 128; }
__host__ __device__ constexpr size_t block_bytes_int4(int d) { return (size_t)20 * d; }
__host__ __device__ inline size_t block_offset(int page, int head, int num_pages, size_t bb) {
  return ((size_t)head * num_pages + page) * bb;
}

// ---- device helpers ---------------------------------------------------------

// Rust `as i32` from f32: NaN -> 0, saturating, truncating.
__device__ __forceinline__ int32_t sat_i32(float x) {
  if (x != x) return 0;
  if (x >= 2147483648.0f) return INT32_MAX;
  if (x <= -2147483648.0f) return INT32_MIN;
  return (int32_t)x;
}

// Rust `as u32` from f32: NaN -> 0, negative -> 0, saturating, truncating.
__device__ __forceinline__ uint32_t sat_u32(float x) {
  if (x != x) return 0u;
  if (x <= 0.0f) return 0u;
  if (x >= 4294967296.0f) return 0xFFFFFFFFu;
  return (uint32_t)x;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

// f32 -> bf16 bits, round to nearest even; a NaN stays a quiet NaN of the same
// sign (f32_to_bf16, onnx-rt/src/tensor.rs:312-329).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float v) {
  const uint32_t bits = __float_as_uint(v);
  if (v != v) return (uint16_t)((bits >> 16) | 0x0040u);
  return (uint16_t)((bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16);
}

// Element idx of an attention output of f32, or of bf16 when out_bf16.
__device__ __forceinline__ void store_out(void* out, size_t idx, float v, int out_bf16) {
  if (out_bf16)
    ((uint16_t*)out)[idx] = f32_to_bf16_rne(v);
  else
    ((float*)out)[idx] = v;
}

// Element i of an f32 or bf16 row (base 4-byte aligned). Branch-free: one
// dword load for either type, so a run of these issues back to back instead
// of waiting at the join of two load paths.
__device__ __forceinline__ float load_elem(const void* base, size_t i, int dtype) {
  const bool h = dtype == kDtypeBf16;
  const uint32_t w = ((const uint32_t*)base)[h ? (i >> 1) : i];
  return __uint_as_float(h ? ((i & 1) ? (w & 0xFFFF0000u) : (w << 16)) : w);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// v_min_f32 / v_max_f32 whose first operand is read from another lane of the
// row by DPP (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror). Their operands are values that are never signalling NaNs
// (results of arithmetic, min or max), so the quieting step the compiler puts
// before fminf / fmaxf of a DPP move is not needed. The s_nop covers the wait
// states between a VALU write of the source (or of EXEC) and its DPP read.
#define SAI_DPP_OP(name, op, ctrl)                                                   \
  __device__ __forceinline__ float name(float a) {                                  \
    float r;                                                                         \
    asm("s_nop 4\n\t" op " %0, %1, %1 " ctrl " row_mask:0xf bank_mask:0xf"        \
        : "=v"(r)                                                                    \
        : "v"(a));                                                                   \
    return r;                                                                        \
  }
SAI_DPP_OP(min_quad1032, "v_min_f32_dpp", "quad_perm:[1,0,3,2]")
SAI_DPP_OP(max_quad1032, "v_max_f32_dpp", "quad_perm:[1,0,3,2]")
SAI_DPP_OP(min_quad2301, "v_min_f32_dpp", "quad_perm:[2,3,0,1]")
SAI_DPP_OP(max_quad2301, "v_max_f32_dpp", "quad_perm:[2,3,0,1]")
SAI_DPP_OP(min_half_mirror, "v_min_f32_dpp", "row_half_mirror")
SAI_DPP_OP(max_half_mirror, "v_max_f32_dpp", "row_half_mirror")
SAI_DPP_OP(max_row_mirror, "v_max_f32_dpp", "row_mirror")
#undef SAI_DPP_OP

// The largest value of the wave, in every lane, for values that are never
// signalling NaNs. The max is exact, so the order of the steps does not change
// it: DPP within each row of 16 lanes (the quads, the halves, the row), then
// the gfx950 row swaps (swap(x, x) leaves the lane's own value in one result
// and its partner's in the other, so their max needs no select).
__device__ __forceinline__ float max2_f32(float a, float b) {
  float r;
  asm("v_max_f32_e32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float wave_max_rows(float v) {
  v = max_quad1032(v);
  v = max_quad2301(v);
  v = max_half_mirror(v);
  v = max_row_mirror(v);
  const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
  v = max2_f32(__uint_as_float(s16[0]), __uint_as_float(s16[1]));
  const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
  return max2_f32(__uint_as_float(s32[0]), __uint_as_float(s32[1]));
}

// ---- launch parameters --------------------------------------------------------

struct AppendParams {
  const void* k;  // [batch, s_new, Hkv*D]
  const void* v;
  int dtype;
  int batch, s_new, kv_heads;
  const float* cos_cache;
  const float* sin_cache;
  int cache_rows;
  int do_rotary, interleaved;
  const int32_t* seq_lens;    // device [batch] committed lengths
  const int32_t* page_table;  // device [batch][max_pages]
  int max_pages;
  uint8_t* pool;
  int num_pages;
  // pages the new tokens touch in the sequence that touches most (the page
  // kernel's grid); 0: s_new / 16 + 1, which covers any start
  int pages;
};

// Sequences whose work items a ragged decode launch can order (longest
// splits first); the order rides in the kernel arguments.
constexpr int kDecodeOrder = 256;

struct DecodeParams {
  const void* q;  // [batch, 1, Hq*D]
  int q_dtype;
  void* out;     // [batch, 1, Hq*D], f32 or (out_bf16) bf16
  int out_bf16;
  const uint8_t* pool;
  int kv_heads, num_pages;
  const int32_t* seq_lens;  // device [batch] committed
  int pending;              // attention length = seq_lens[b] + pending
  const int32_t* page_table;
  int max_pages;
  int batch;
  const float* cos_cache;
  const float* sin_cache;
  int cache_rows, do_rotary, interleaved;
  float scale_log2;   // softmax scale * log2(e)
  int split_tokens;   // tokens per workgroup, multiple of 64
  int waves;          // waves per workgroup (4 or 8)
  int uniform_nsplit; // > 0: every sequence has this many splits (no scan)
  int max_nsplit;     // the largest split count of any sequence
  float* partials;    // [work_items * Hkv][G][D + 2]
  int32_t* seq_info;  // [batch][2]: first work item, number of splits
  int merge_in_kernel;  // 1: last workgroup merges the splits (counters)
  int32_t* counters;    // [batch * Hkv], zero between launches
  const void* k_new;    // fused append: [batch, 1, Hkv*D] pre-RoPE K, or null
  const void* v_new;
  int kv_dtype;
  int window;           // visible keys per query (0: all); see window_first_key
  int static_tiles;     // 1: fixed tile order per wave (bit-reproducible output)
  // ragged launches (uniform_nsplit == 0) with batch <= kDecodeOrder: work
  // items go to the sequences in this order (ordered != 0), each sequence's
  // splits in turn
  int ordered;
  uint16_t order[kDecodeOrder];
};

struct PrefillParams {
  const void* q;  // [batch, sq, Hq*D]
  int q_dtype;
  void* out;     // [batch, sq, Hq*D], f32 or (out_bf16) bf16
  int out_bf16;
  const uint8_t* pool;
  int kv_heads, num_pages;
  const int32_t* seq_lens;  // committed; total = seq_lens[b] + sq, queries at seq_lens[b] + i
  int sq;
  const int32_t* page_table;
  int max_pages;
  int batch;
  const float* cos_cache;
  const float* sin_cache;
  int cache_rows, do_rotary, interleaved;
  float scale_log2;
  int window;  // visible keys per query (0: all)
  // one int per workgroup (prefill_workgroups), zero between launches: the
  // int8 fast pass flags the workgroups the precise pass recomputes
  int32_t* prec_flags;
  // key split (nksplit > 1): each workgroup takes ksplit_tiles 64-token tiles
  // of its rows' visible range and writes (m, l, o) partials in the decode's
  // layout (row (b, i) as sequence b * sq + i, nksplit splits each), which the
  // decode's combine kernel merges
  int nksplit, ksplit_tiles;
  float* partials;
};

// Sliding windows: a query at position L-1 sees keys [L - W, L-1] (W > 0)
// or all keys (W == 0). The decode splits of a sequence start at the tile
// (64 tokens) holding its first visible key.
__host__ __device__ inline int window_first_key(int L, int W) { return W > 0 && L > W ? L - W : 0; }
__host__ __device__ inline int window_origin(int L, int W) { return (window_first_key(L, W) / 64) * 64; }

// Positions carried by one rotary launch (kernel argument block).
constexpr int kRotaryTab = 512;

// One launch of the standalone rotary kernel over sequences [b0, b0 + nb) and
// sequence indices [s0, s0 + ns) (nb is implied by total). Rows of head_dim
// elements: layout 0 = (b, h, s) order ([B, H, S, D]), 1 = (b, s, h) order
// ([B, S, H*D]). Position of row (b, s): mode 0: tab[b - b0] + s, mode 1:
// tab[s - s0]. A (b, s) step has head_groups groups of heads_per_item heads
// (the last one may be short), each with `items` work items: rot_items
// rotation items of pairs_per_item pairs, then (out of place) pass-through
// items of pairs_per_item elements from rot_dim on. Supported
// (pairs_per_item, heads_per_item): (1, 1), (4, 4), (8, 2).
struct RotaryArgs {
  const void* x;
  void* y;
  const void* cos;
  const void* sin;
  uint32_t total;  // work items of the launch
  int32_t items, rot_items, pairs_per_item, heads_per_item, head_groups;
  int32_t heads, seq, head_dim, rot_dim, cache_cols;
  int32_t layout, mode;
  int32_t b0, s0, ns;
  int32_t tab[kRotaryTab];
};

// Row copy (copy_rows.hip): src holds batch x heads x seq rows of
// `chunks` chunks in src_layout (0: (b, h, s) order, 1: (b, s, h)); row
// (b, h, s) goes to row (b, h, dst_offset + s) of dst, which holds dst_seq
// sequence positions in dst_layout.
struct CopyRowsArgs {
  const void* src;
  void* dst;
  uint64_t total;  // rows * chunks
  int32_t chunks;  // chunks per row
  int32_t heads, seq, dst_seq, dst_offset;
  int32_t src_layout, dst_layout;
};

// TurboQuant cache, one layer (tq_cache.hip). Row (head h, sequence b,
// position r) = (h * batch_cap + b) * rows_cap + r of the row-major arrays:
//   K codes   [row][code_stride bytes], packed LSB first along head_dim
//   par_k/v   [row] float4 (scale, zero point, QJL mean, sum of the codes)
//   signs_k/v [row][D/32] QJL sign words (bit i of word j: dim 32j + i)
// V codes are tile-transposed for the PV product: tile = 64 positions of one
// (h, b), at ((h * batch_cap + b) * tiles_cap + r / 64) * tq_vtile_bytes;
// inside it dim d owns 64 * bits bits (8 * bits bytes) holding the codes of
// the tile's 64 positions, position r % 64 at bit (r % 64) * bits, LSB first.
__host__ __device__ constexpr size_t tq_vtile_bytes(int d, int bits) {
  return (size_t)d * 8 * bits;
}

struct TqArgs {
  uint8_t* codes_k;
  uint8_t* codes_v;
  float4* par_k;
  float4* par_v;
  uint32_t* signs_k;
  uint32_t* signs_v;
  const int8_t* signs;       // rotation signs [heads][D] of this layer
  const int32_t* seq_lens;   // committed rows per sequence
  int pending;
  int heads, batch_cap, rows_cap, tiles_cap, head_dim, bits, qjl;
  size_t code_stride;  // bytes per row of K codes (multiple of 16)
  float norm;          // 1 / sqrt_approx(head_dim)
  // low-rank K (rank 1), null when the cache keeps none: U_S per row
  // [heads][batch_cap][rows_cap], Vt [heads][batch_cap][D], and the
  // re-decomposition's u vector, laid out as U_S
  float* lr_us;
  float* lr_vt;
  float* lr_u;
};

struct TqAttendArgs {
  const void* q;  // [batch, 1, num_heads * D]
  int q_bf16;
  int num_heads;
  float* out;       // [batch, 1, num_heads * D]
  float* partials;  // [batch][heads][max_splits][G * (D + 2)]
  int* counters;    // [batch][heads] split tickets, zero between launches
  const float* weights;  // weighted value sum: [batch * num_heads][ld]
  int ld;                // row stride of logits / weights
  int normalize;         // 0: the weighted sum is not divided by the weights' sum
  const void* k_new;     // fused step: the pass's new row per (sequence, kv head),
  const void* v_new;     //   [batch, 1, heads * D], stored before it is attended
  int kv_bf16;
  int split_rows, max_splits;  // max_splits: the launch grid's splits per sequence
  float scale_log2;
  int static_tiles;  // 1: fixed tile order per wave (bit-reproducible output)
};

// Launchers (return hipError_t of the launch).
hipError_t launch_tq_write(const TqArgs& a, const void* k, const void* v, int bf16, int batch,
                           int s_new, hipStream_t st);
hipError_t launch_tq_lowrank(const TqArgs& a, const void* k, int bf16, int batch, int s_new,
                             hipStream_t st);
hipError_t launch_tq_read(const TqArgs& a, int b, int h, int start, int len, float* k_out,
                          float* v_out, hipStream_t st);
// mode 0 attention, 1 logits only, 2 weighted value sum only
hipError_t launch_tq_attend(const TqArgs& a, const TqAttendArgs& t, int mode, int group,
                            int nsplit, int batch, hipStream_t st);
hipError_t launch_copy_rows(const CopyRowsArgs& a, int chunk_bytes, hipStream_t st);
// p[0, n) = v on the stream (a kernel, so that graph capture records no memset
// node; copy_rows.hip).
hipError_t launch_fill_i32(int32_t* p, size_t n, int32_t v, hipStream_t st);
// Standalone RoPE (rotary.hip): x/y f32 or bf16, tables f32 or bf16.
hipError_t launch_rotary(const RotaryArgs& a, bool x_bf16, bool table_bf16, bool interleaved,
                         hipStream_t st);
// RoPE tables [max_pos, half] of the Gemma loader's precompute (rotary.hip),
// bf16 or (bf16 values widened to) f32.
hipError_t launch_rope_tables(float theta, uint32_t max_pos, uint32_t half, bool bf16,
                              void* cos_out, void* sin_out, hipStream_t st);
hipError_t launch_kv_append(const AppendParams& p, int head_dim, int quant, hipStream_t s);
hipError_t launch_gqa_decode(const DecodeParams& p, int head_dim, int group, int quant,
                             int work_items, bool combine, hipStream_t s);
hipError_t launch_gqa_prefill(const PrefillParams& p, int head_dim, int group, int quant,
                              hipStream_t s);
// Workgroups of one prefill launch (the size of PrefillParams::prec_flags).
size_t prefill_workgroups(const PrefillParams& p, int head_dim, int group);
// Split-partial merge of the decode kernels (gqa_decode.hip).
hipError_t launch_decode_combine(const DecodeParams& p, int head_dim, int group, hipStream_t st);
// int4 decode (gqa_decode_int4.hip): head_dim 128; merges through the combine
// kernel when `combine` and a sequence has several splits.
hipError_t launch_gqa_decode_int4(const DecodeParams& p, int head_dim, int group, int work_items,
                                  bool combine, hipStream_t st);
hipError_t launch_seq_advance(int32_t* seq_lens, int batch, int pending, hipStream_t s);

}  // namespace sai
