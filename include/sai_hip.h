/*
 * libsai_hip -- C ABI of the MI355X (gfx950) compressed-KV
 * GroupQueryAttention path.
 *
 * This is the drop-in boundary for SmallAIOS onnx-rt's
 * com.microsoft.GroupQueryAttention with fused rotary embedding over a
 * quantised, paged KV cache. Plain C: integers, floats and raw pointers only.
 * Every device pointer is caller-owned unless a function says otherwise; no
 * C++ exception crosses the boundary; every call is asynchronous on the given
 * HIP stream (void* = hipStream_t, NULL = the null stream) unless documented
 * as synchronous.
 *
 * Each entry point names the reference interface it replaces
 * (paths relative to the SmallAIOS workspace root).
 *
 * Threading: a sai_ctx and the caches created from it are thread-compatible,
 * not thread-safe. The reference holds its cache behind Arc<Mutex<_>>
 * (onnx-rt/src/session.rs:377); callers do the same.
 *
 * Streams: each cache (sai_kvcache, sai_tqcache) owns the device scratch its
 * attention launches use, sized when it is created (a launch that needs more,
 * such as a prefill chunk's key split, grows it once, synchronously), so
 * different caches may run on different streams at once. The launches on one cache must be
 * ordered by the caller (one stream, or events between streams), as the
 * cache's contents already require. Calls documented as synchronous wait for
 * all work on the device first.
 */
#ifndef SAI_HIP_H
#define SAI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. The negative codes mirror the reference's error variants:
 * OpError::{InvalidAttribute, ShapeMismatch, UnsupportedOp}
 * (onnx-rt/src/operators.rs:26-37) and CudaError::{RuntimeError, AllocFailed}
 * plus the cache's "position_overflow" (onnx-rt/src/cuda/kv_cache.rs:245-250). */
typedef int32_t sai_status;
#define SAI_OK 0
#define SAI_ERR_INVALID_ATTRIBUTE (-1)
#define SAI_ERR_SHAPE_MISMATCH (-2)
#define SAI_ERR_UNSUPPORTED (-3)
#define SAI_ERR_HIP (-4)
#define SAI_ERR_ALLOC (-5)
#define SAI_ERR_OVERFLOW (-6)
#define SAI_ERR_NULL (-7)

/* Element types, numbered as the reference's DataType / ONNX TensorProto
 * (onnx-rt/src/tensor.rs). */
#define SAI_DTYPE_F32 1
#define SAI_DTYPE_F16 10
#define SAI_DTYPE_BF16 16

/* KV quantisation schemes.
 * INT8: symmetric, one f32 scale per (token, kv head): s = amax/127 (1.0 when
 *       amax == 0), code = clamp(round_half_even(x/s), -128, 127)
 *       (QuantizeLinear semantics, onnx-rt/src/ops/quantized.rs:115-164).
 * INT4: asymmetric per (token, kv head, group of 32 along head_dim): min/max
 *       quantiser of onnx-rt/src/kv_compression.rs:223-253 with levels 15,
 *       scale and zero point stored as IEEE binary16, codes packed LSB-first
 *       (kv_compression.rs:294-312). */
#define SAI_KV_INT8 1
#define SAI_KV_INT4 2

/* Tokens per cache page. */
#define SAI_PAGE_TOKENS 16

typedef struct sai_ctx sai_ctx;
typedef struct sai_kvcache sai_kvcache;

/* ---- runtime --------------------------------------------------------------
 * Replaces CudaRuntime::new / drop (onnx-rt/src/cuda/mod.rs:619-700). */
sai_status sai_init(int device, sai_ctx** out);
void sai_destroy(sai_ctx* ctx);
/* Message of the last failed call on ctx ("" if none). Valid until the next
 * call on ctx. Replaces the Display of CudaError/OpError. */
const char* sai_last_error(const sai_ctx* ctx);
/* 1 / sqrt(head_dim) computed exactly as the reference's default GQA scale
 * (Newton sqrt_f32, onnx-rt/src/ops/microsoft.rs:54-63 and :1153). */
float sai_default_scale(int32_t head_dim);
/* Device kernels are compiled for gfx950 only; returns 1 when `device` is one. */
int32_t sai_device_supported(int device);

/* ---- paged quantised KV cache ---------------------------------------------
 * Replaces GpuKvCache (onnx-rt/src/cuda/kv_cache.rs:111-390). Differences by
 * design: pages of SAI_PAGE_TOKENS tokens behind a per-sequence page table
 * instead of one linear [max_seq, Hkv, D] buffer, a committed length per
 * sequence instead of one current_position, and int8/int4 codes instead of
 * bf16. Lifecycle is the reference's: append (pending, not committed) ->
 * attention sees committed + pending tokens (view_pending, kv_cache.rs:320) ->
 * advance once per forward pass (advance_position, kv_cache.rs:295). */
typedef struct sai_kvcache_desc {
  int32_t num_layers;
  int32_t num_kv_heads;
  int32_t head_dim;          /* 64, 128, 256, or 168 for int8 (Gemma 4 31B); int4
                                decode: groups up to 4 at 256 */
  int32_t num_pages;         /* physical pages per layer */
  int32_t max_batch;         /* sequences */
  int32_t max_pages_per_seq; /* page-table width */
  int32_t quant;             /* SAI_KV_INT8 or SAI_KV_INT4 */
} sai_kvcache_desc;

/* Allocates num_layers pools of num_pages pages (zero-filled, as
 * GpuKvCache::allocate zero-fills, kv_cache.rs:176-179). Synchronous.
 * Errors: SHAPE_MISMATCH for zero/unsupported dims (kv_cache_allocate:zero_dim),
 * ALLOC when device memory runs out. */
sai_status sai_kvcache_create(sai_ctx* ctx, const sai_kvcache_desc* desc, sai_kvcache** out);
void sai_kvcache_destroy(sai_kvcache* cache);

/* Page table for `batch` sequences, host array [batch][max_pages_per_seq] of
 * physical page ids in [0, num_pages), or -1 for an unmapped slot. Every entry
 * is validated on the host. Synchronous. Resets all lengths to 0. */
sai_status sai_kvcache_set_page_table(sai_ctx* ctx, sai_kvcache* cache, const int32_t* page_table,
                                      int32_t batch);
/* Committed lengths (host array [batch]); clears pending tokens. Synchronous. */
sai_status sai_kvcache_set_seq_lens(sai_ctx* ctx, sai_kvcache* cache, const int32_t* seq_lens,
                                    int32_t batch);
/* Commit the pending tokens of the current forward pass: every committed
 * length grows by the pending count. Stream-ordered. Replaces
 * GpuKvCache::advance_position (kv_cache.rs:295-304). */
sai_status sai_kvcache_advance(sai_ctx* ctx, sai_kvcache* cache, void* stream);
/* Layer kind (LayerKind, kv_cache.rs:53-60): window > 0 makes `layer` a
 * sliding-window layer whose queries see only their last `window` keys
 * (GpuKvCache::view_at, kv_cache.rs:340-360); 0 = global (the default). The
 * pages keep every token; only attention is limited. Host-side. */
sai_status sai_kvcache_set_layer_window(sai_ctx* ctx, sai_kvcache* cache, int32_t layer,
                                        int32_t window);
/* All lengths back to 0, buffers kept (GpuKvCache::reset, kv_cache.rs:386-388). */
sai_status sai_kvcache_reset(sai_ctx* ctx, sai_kvcache* cache);
/* Host view of the lengths: seq_lens_out[batch] (committed), *pending_out. */
sai_status sai_kvcache_lengths(const sai_kvcache* cache, int32_t* seq_lens_out,
                               int32_t* pending_out, int32_t* batch_out);
/* Copy n_tokens tokens [t0, t0+n_tokens) of (sequence b, kv head h, layer) out
 * of the pages into host buffers in logical order. Synchronous (debug,
 * checkpoint and tests). INT8: k/v_codes int8 [n][D], k/v_params f32 [n]
 * scales. INT4: k/v_codes u8 [n][D/2] packed LSB-first along D, k/v_params
 * u16 [n][D/32][2] binary16 (scale, zero). */
sai_status sai_kvcache_read(sai_ctx* ctx, sai_kvcache* cache, int32_t layer, int32_t b,
                            int32_t kv_head, int32_t t0, int32_t n_tokens, void* k_codes,
                            void* v_codes, void* k_params, void* v_params);
/* Raw pool of one layer (device pointer and size in bytes) and the bytes of
 * one (page, kv head) block. Block (page p, kv head h) starts at
 * (h * num_pages + p) * block_bytes; INT8 block: K codes [16][D] int8, V codes
 * [D][16] int8, K scales [16] f32, V scales [16] f32 (32*D + 128 bytes); INT4
 * block: K codes [16][D/2], V codes [D][8] (LSB-first along slots), K then V
 * (scale, zero) binary16 [16][D/32][2] (20*D bytes). D is the stored row
 * width: head_dim, except 192 for head_dim 168, whose dims 0-83 sit at 0-83
 * and 84-167 at 96-179 (split-half RoPE pairs (i, i + 96)), the rest 0.
 * sai_kvcache_read returns the head_dim codes of a row. */
sai_status sai_kvcache_pool(const sai_kvcache* cache, int32_t layer, void** dev_ptr,
                            size_t* bytes, size_t* block_bytes);

/* ---- kernel 1: RoPE + quantise + pack append --------------------------------
 * Replaces GpuKvCache::append (kv_cache.rs:233-278) fused with the K half of
 * gqa_apply_rotary (onnx-rt/src/ops/microsoft.rs:1004-1052) and the
 * QuantizeLinear of the KV scheme. k, v: device [batch, s_new, Hkv*D] of
 * `dtype` (F32 or BF16), pre-RoPE K. Token s of sequence b goes to position
 * seq_len[b] + s; RoPE (when do_rotary) uses that position in cos/sin
 * ([cache_rows, D/2] f32, device, 16-byte aligned; the same tables and
 * alignment for every attention entry point below). Leaves s_new tokens
 * pending; the same s_new must be used for every layer of a forward pass, and
 * appending a layer twice before advance rewrites the same slots.
 * Errors: SHAPE_MISMATCH (dims, unmapped page, position >= cache_rows),
 * OVERFLOW (past the page table), UNSUPPORTED (dtype/head_dim). */
sai_status sai_kv_append(sai_ctx* ctx, sai_kvcache* cache, int32_t layer, const void* k,
                         const void* v, int32_t dtype, int32_t batch, int32_t s_new,
                         const float* cos_cache, const float* sin_cache, int32_t cache_rows,
                         int32_t do_rotary, int32_t rotary_interleaved, void* stream);

/* ---- kernel 2: split-K flash decode -----------------------------------------
 * Replaces gpu_gqa_with_cache (onnx-rt/src/cuda/kernels/attention.rs:1260-1295)
 * and, for Sq == 1, op_group_query_attention's attention half
 * (onnx-rt/src/ops/microsoft.rs:1082-1190): RoPE on Q at position
 * seq_len[b] + pending - 1, causal attention over the committed + pending
 * tokens of each sequence (ragged lengths allowed), GQA head grouping
 * kh = qh / (Hq/Hkv). Requires pending == 1.
 * q: device [batch, 1, num_heads*D] of `dtype` (F32 or BF16);
 * out: device [batch, 1, num_heads*D] of out_dtype: F32, or BF16 rounded to
 * nearest even from the f32 result (the reference's GPU attention returns
 * Q's dtype, attention.rs:835 and :877-901, and the bf16 GEMM after it takes
 * only bf16 x bf16, gpu_executor.rs:1024-1031); UNSUPPORTED otherwise.
 * scale: used when has_scale != 0, else sai_default_scale(D).
 * window: gpu_gqa_with_cache's `window` (the node's local_window_size when
 * > 0): the query at position p sees keys [p - window, p]; <= 0 = off. A
 * sliding-window layer (sai_kvcache_set_layer_window) sees its last w keys;
 * with both, the narrower span applies. Head dims 64, 128 and 256 for int8
 * and int4, and 168 for int8; groups 1, 2, 4 and 8 (int4 at 256: up to 4);
 * UNSUPPORTED otherwise. */
sai_status sai_gqa_decode(sai_ctx* ctx, sai_kvcache* cache, int32_t layer, const void* q,
                          int32_t dtype, int32_t batch, int32_t num_heads,
                          const float* cos_cache, const float* sin_cache, int32_t cache_rows,
                          int32_t do_rotary, int32_t rotary_interleaved, int32_t has_scale,
                          float scale, int32_t window, void* out, int32_t out_dtype,
                          void* stream);

/* ---- kernels 1 + 2 fused: one decode step in one launch ----------------------
 * Replaces gpu_gqa_with_cache (onnx-rt/src/cuda/kernels/attention.rs:1260-1295),
 * which appends the step's K/V to the cache (GpuKvCache::append) and attends
 * over view_pending: here the decode kernel's workgroup that owns a sequence's
 * last split writes the new token (same RoPE/quantise arithmetic as
 * sai_kv_append, bit for bit) before streaming its tiles. k_new, v_new: device
 * [batch, 1, Hkv*D] of kv_dtype (F32 or BF16). Leaves 1 token pending, exactly
 * like sai_kv_append with s_new = 1 followed by sai_gqa_decode. */
sai_status sai_gqa_with_cache(sai_ctx* ctx, sai_kvcache* cache, int32_t layer, const void* q,
                              int32_t q_dtype, const void* k_new, const void* v_new,
                              int32_t kv_dtype, int32_t batch, int32_t num_heads,
                              const float* cos_cache, const float* sin_cache, int32_t cache_rows,
                              int32_t do_rotary, int32_t rotary_interleaved, int32_t has_scale,
                              float scale, int32_t window, void* out, int32_t out_dtype,
                              void* stream);

/* ---- the fused decode step without allocation ---------------------------------
 * No counterpart in the reference: this is for callers that cannot allocate
 * device memory during a step (code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation). Same contract, arguments and
 * results as sai_gqa_with_cache, but the step's scratch (split partials,
 * split ranges, merge tickets) lives in one fixed 16 MiB array per GPU that
 * the library sets up in sai_init and holds until the process ends, instead
 * of the cache's own workspace; nothing is allocated or freed. Limits: at
 * most 65536 (sequence x kv head) pairs, 32768 sequences, and 4,063,232
 * partial floats, i.e. sequence-splits x kv heads x group x (D + 2), D the
 * stored row width (sai_kvcache_pool)
 * (the Llama-3-8B layer at 16 x 8k uses 133,120); a larger step fails with
 * UNSUPPORTED. Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (other streams, other threads, other contexts) race, and
 * their outputs are undefined. Each call first clears its merge tickets with
 * a small fill kernel on `stream` (no memset node under graph capture), so
 * what a racing call left behind does not reach the calls after it. */
sai_status sai_gqa_with_cache_noalloc(sai_ctx* ctx, sai_kvcache* cache, int32_t layer,
                                      const void* q, int32_t q_dtype, const void* k_new,
                                      const void* v_new, int32_t kv_dtype, int32_t batch,
                                      int32_t num_heads, const float* cos_cache,
                                      const float* sin_cache, int32_t cache_rows,
                                      int32_t do_rotary, int32_t rotary_interleaved,
                                      int32_t has_scale, float scale, int32_t window, void* out,
                                      int32_t out_dtype, void* stream);

/* ---- kernel 3: prefill chunk (f16 MFMA) ---------------------------------------
 * Same contract as sai_gqa_decode for a chunk of sq == pending query tokens per
 * sequence (the reference's op_group_query_attention with Sq > 1, causal with
 * past_sk = seq_len[b], microsoft.rs:1156 and :331-337), over an int8 cache
 * (head_dim 64, 128, 168 or 256) or an int4 one (head_dim 64, 128 or 256).
 * q: device [batch, sq, num_heads*D]; out: device [batch, sq, num_heads*D] of
 * out_dtype (F32 or BF16, as for sai_gqa_decode).
 * window and sliding-window layers as for sai_gqa_decode, applied to every
 * query row at its own position (gpu_gqa's mask, attention.rs:79, :111).
 * A short chunk over a long past is split over the key range: partials in the
 * cache's decode workspace, merged by a second kernel on the same stream (the
 * workspace grows once, synchronously, when a shape needs more). */
sai_status sai_gqa_prefill(sai_ctx* ctx, sai_kvcache* cache, int32_t layer, const void* q,
                           int32_t dtype, int32_t batch, int32_t sq, int32_t num_heads,
                           const float* cos_cache, const float* sin_cache, int32_t cache_rows,
                           int32_t do_rotary, int32_t rotary_interleaved, int32_t has_scale,
                           float scale, int32_t window, void* out, int32_t out_dtype,
                           void* stream);

/* ---- standalone rotary embedding ----------------------------------------------
 * Replaces op_rotary_embedding (onnx-rt/src/ops/microsoft.rs:556-652, through
 * apply_rope_in_place :177-233 and validate_rope_caches :71-110) and
 * rotary_gpu (onnx-rt/src/cuda/kernels/rotary.rs:274-374).
 * x, y: device, batch*num_heads*seq rows of head_dim elements of `dtype`
 * (F32 or BF16); y == x rotates in place, otherwise y must not overlap x and
 * the elements at and past rotary_dim are copied to y unchanged. Row order:
 *   SAI_ROPE_BHSD: rows (b, h, s) of [batch, num_heads, seq, head_dim] (also
 *                  op_rotary_embedding's view of a rank-3 [B, S, H*D] buffer,
 *                  which it reinterprets without a transpose);
 *   SAI_ROPE_BSHD: rows (b, s, h) of [batch, seq, num_heads*head_dim]
 *                  (rotary_gpu's rank-3 layout).
 * Positions: position_ids (HOST memory) of n_pos == seq entries (shared by all
 * sequences; tested first) or n_pos == batch*seq (row b*seq + s); or, with
 * position_ids == NULL, start_position + s for every sequence (rotary_gpu).
 * cos/sin: device [cache_rows, cache_cols] of table_dtype (F32, or BF16 read
 * as its exact f32 value); cache_cols must equal rotary_dim / 2.
 * rotary_dim: <= 0 means head_dim; must be even and at most head_dim.
 * Pairs (i, i + rotary_dim/2), or (2i, 2i+1) when interleaved; y0 = c*x0 - s*x1,
 * y1 = s*x0 + c*x1 in f32 with each product rounded on its own; BF16 output
 * rounds to nearest even.
 * Errors: SHAPE_MISMATCH (negative dims, n_pos, cache_cols, a position outside
 * [0, cache_rows), missing tables), INVALID_ATTRIBUTE (rotary_dim, layout),
 * UNSUPPORTED (dtype, or one (b, s) step larger than 2^31 work items). */
#define SAI_ROPE_BHSD 0
#define SAI_ROPE_BSHD 1
sai_status sai_rotary_embedding(sai_ctx* ctx, const void* x, void* y, int32_t dtype, int32_t batch,
                                int32_t num_heads, int32_t seq, int32_t head_dim, int32_t layout,
                                const int64_t* position_ids, int64_t n_pos,
                                int64_t start_position, const void* cos_cache,
                                const void* sin_cache, int32_t table_dtype, int32_t cache_rows,
                                int32_t cache_cols, int32_t rotary_dim, int32_t interleaved,
                                void* stream);

/* ---- row copy between layouts ------------------------------------------------
 * Replaces kv_concat / kv_copy_block (onnx-rt/src/ops/microsoft.rs:733-792) and
 * reshape_to_bhsd / reshape_from_bhsd (microsoft.rs:660-704): src holds
 * batch*heads*seq rows of head_dim elements of `dtype` (F32 or BF16) in
 * src_layout; row (b, h, s) is copied to row (b, h, dst_offset + s) of dst,
 * which holds dst_seq positions per (b, h) in dst_layout (SAI_ROPE_BHSD =
 * [B, H, S, D], SAI_ROPE_BSHD = [B, S, H*D]). A past K/V [B, H, P, D] and a
 * step's new rows [B, S, H*D] concatenate into present [B, H, P+S, D] with two
 * calls. src and dst must not overlap. Errors: SHAPE_MISMATCH (the rows do not
 * fit dst), INVALID_ATTRIBUTE (layout), UNSUPPORTED (dtype). */
sai_status sai_copy_rows(sai_ctx* ctx, const void* src, int32_t src_layout, void* dst,
                         int32_t dst_layout, int32_t dtype, int32_t batch, int32_t heads,
                         int32_t seq, int32_t head_dim, int32_t dst_seq, int32_t dst_offset,
                         void* stream);

/* ---- RoPE tables ---------------------------------------------------------------
 * Replaces precompute_rope_tables (onnx-rt/src/model_loader/gemma.rs:458-472)
 * with its f32 approximations powf/ln/exp/floor/sin/cos (gemma.rs:480-541):
 * row pos, column i: inv_freq = 1 / powf_approx(rope_theta, 2i / (2*half)),
 * angle = pos * inv_freq, cos_approx / sin_approx of angle rounded to bf16;
 * bit for bit the reference's tables. cos_out, sin_out: device
 * [max_pos, half] of dtype BF16, or F32 (the same bf16 values widened, as the
 * reference's GPU dispatch casts them). Errors: UNSUPPORTED (dtype,
 * max_pos*half >= 2^31), SHAPE_MISMATCH (negative sizes). */
sai_status sai_rope_tables(sai_ctx* ctx, float rope_theta, int32_t max_pos, int32_t half,
                           int32_t dtype, void* cos_out, void* sin_out, void* stream);

/* ---- TurboQuant compressed KV cache -------------------------------------------
 * Replaces CompressedKVCache (onnx-rt/src/kv_compression.rs:738-963, with
 * kv_lowrank_k = None) on the device, plus the decode read path of its design
 * (docs/kv-compression-design.md section 9). Each row (token, kv head) of K
 * and of V is PolarQuant-encoded with the head's quantizer (xorshift64 signs
 * seeded seed * 0x9E3779B97F4A7C15 + layer * num_kv_heads + head, normalised
 * Walsh-Hadamard rotation, one min/max quantiser of `bits` bits over the
 * rotated row) and, with qjl, its QJL residual (sign bits of x - decode, mean
 * |residual|); codes, scale, zero point, sign bits and mean are the
 * reference's bit for bit. Every sequence of a pass appends the same number
 * of rows (pending until sai_tqcache_advance), as the paged cache does. */
typedef struct sai_tqcache sai_tqcache;
typedef struct sai_tqcache_desc {
  int32_t num_layers;
  int32_t num_kv_heads;
  int32_t head_dim;  /* 64, 128 or 256 (attention groups up to 4 at 256) */
  int32_t bits;      /* 3, 4 or 8 (kv_quant_bits) */
  int32_t qjl;       /* kv_qjl_residual */
  int32_t max_batch; /* sequences */
  int32_t max_rows;  /* rows per sequence */
  uint64_t seed;     /* KVCacheConfig::seed */
  /* kv_lowrank_k: 0 = None; r >= 1 = Some(r) (Some(0) means Some(1),
   * LowRankKeyDecomposer::new, kv_compression.rs:461-465). The cache
   * decomposes each head's first K row alone, so the kept rank is 1 for any
   * r (:840-852); read_k then reconstructs K from it. */
  int32_t lowrank_k;
} sai_tqcache_desc;
/* Allocates the layers' storage and uploads the rotation signs. Synchronous.
 * Errors: SHAPE_MISMATCH (zero sizes), UNSUPPORTED (head_dim),
 * INVALID_ATTRIBUTE ("bits must be 3, 4, or 8"), ALLOC. */
sai_status sai_tqcache_create(sai_ctx* ctx, const sai_tqcache_desc* desc, sai_tqcache** out);
void sai_tqcache_destroy(sai_tqcache* cache);
/* CompressedKVCache::write_kv for every kv head of `layer`: k, v device
 * [batch, s_new, num_kv_heads*head_dim] (F32 or BF16) become rows
 * len[b] .. len[b] + s_new - 1 (pending); a low-rank K takes the rows in
 * order (LowRankKeyDecomposer decompose / update, :840-852), once per layer
 * and pass. Errors: SHAPE_MISMATCH (layer, sizes, a pass mixing row counts),
 * OVERFLOW (past max_rows), UNSUPPORTED (dtype; a layer's low-rank K written
 * twice in one pass). */
sai_status sai_tqcache_write(sai_ctx* ctx, sai_tqcache* cache, int32_t layer, const void* k,
                             const void* v, int32_t dtype, int32_t batch, int32_t s_new,
                             void* stream);
/* Commit the pending rows (one call per pass; none pending: no-op).
 * Stream-ordered. */
sai_status sai_tqcache_advance(sai_ctx* ctx, sai_tqcache* cache, void* stream);
/* Committed lengths of sequences 0..batch-1 (<= max_rows; rows beyond a
 * length are ignored), dropping anything pending; the next pass has `batch`
 * sequences. Synchronous. Errors: SHAPE_MISMATCH, OVERFLOW, UNSUPPORTED (a
 * low-rank K, whose state follows the rows written: use reset). */
sai_status sai_tqcache_set_lengths(sai_ctx* ctx, sai_tqcache* cache, const int32_t* lens,
                                   int32_t batch);
/* All lengths back to 0 (storage kept). Synchronous. */
sai_status sai_tqcache_reset(sai_ctx* ctx, sai_tqcache* cache);
/* Host view: lens_out[max_batch] committed rows, *pending_out, *batch_out. */
sai_status sai_tqcache_lengths(const sai_tqcache* cache, int32_t* lens_out, int32_t* pending_out,
                               int32_t* batch_out);
/* memory_bytes (kv_compression.rs:928-957): *reference_bytes = the
 * reference's accounting of the committed rows (every layer holding each
 * sequence's rows: packed codes + 25 bytes per block, sign words + 12 bytes
 * per residual, K and V); *device_bytes = what this cache holds on the
 * device at its capacity. Either may be NULL. */
sai_status sai_tqcache_memory_bytes(const sai_tqcache* cache, uint64_t* reference_bytes,
                                    uint64_t* device_bytes);
/* read_k / read_v (kv_compression.rs:862-907): rows [start, start+len) of
 * (layer, sequence b, kv head) decoded to f32, host arrays [len][head_dim]
 * each; with a low-rank K, k_out is its reconstruction 0 + U_S[t] Vt, as
 * read_k prefers it. Synchronous. */
sai_status sai_tqcache_read(sai_ctx* ctx, sai_tqcache* cache, int32_t layer, int32_t b,
                            int32_t head, int32_t start, int32_t len, float* k_out,
                            float* v_out);
/* The stored form of the same rows (host, any output may be NULL): codes
 * [len][head_dim*bits/8] packed LSB first, params [len][3] f32 (scale,
 * zero point, QJL mean), QJL sign words [len][head_dim/64] u64 (qjl only).
 * Synchronous. */
/* The low-rank K state of (layer, sequence b, kv head) (LowRankK,
 * kv_compression.rs:425-438, rank 1): u_s [len] = U_S of rows
 * [start, start+len), vt [head_dim] (either may be NULL). Synchronous.
 * Errors: UNSUPPORTED (no low-rank K), SHAPE_MISMATCH. */
sai_status sai_tqcache_read_lowrank(sai_ctx* ctx, sai_tqcache* cache, int32_t layer, int32_t b,
                                    int32_t head, int32_t start, int32_t len, float* u_s,
                                    float* vt);
sai_status sai_tqcache_read_raw(sai_ctx* ctx, sai_tqcache* cache, int32_t layer, int32_t b,
                                int32_t head, int32_t start, int32_t len, void* k_codes,
                                void* v_codes, float* k_params, float* v_params, void* k_signs,
                                void* v_signs);
/* Decode attention over the committed + pending rows of `layer`: for query
 * head h (kv head h / (num_heads / num_kv_heads)) the logit of row t is the
 * module's inner-product estimate <decode(q), decode(k_t)> + (qjl ?
 * correction(residual(q), residual(k_t)) : 0) (kv_compression.rs:1254-1288),
 * evaluated on the codes in the rotated domain; softmax(scale * logits); out
 * = sum_t w_t decode(v_t), rotated back once. q: device [batch, 1,
 * num_heads*head_dim] (F32 or BF16); out: device f32, same shape; scale when
 * has_scale, else sai_default_scale(head_dim). */
sai_status sai_tqcache_attend(sai_ctx* ctx, sai_tqcache* cache, int32_t layer, const void* q,
                              int32_t dtype, int32_t batch, int32_t num_heads, int32_t has_scale,
                              float scale, float* out, void* stream);

/* The decode step in one launch (the design's steps 2-6): sai_tqcache_write
 * of one row per sequence (k_new, v_new [batch, 1, num_kv_heads*head_dim],
 * F32 or BF16; pending as after sai_tqcache_write) and sai_tqcache_attend
 * over the rows including it. The workgroup that attends a sequence's last
 * positions stores its new row first. Errors: those of the two calls. */
sai_status sai_tqcache_write_attend(sai_ctx* ctx, sai_tqcache* cache, int32_t layer,
                                    const void* q, int32_t q_dtype, const void* k_new,
                                    const void* v_new, int32_t kv_dtype, int32_t batch,
                                    int32_t num_heads, int32_t has_scale, float scale, float* out,
                                    void* stream);
/* The design's two cache primitives of the GQA read path
 * (docs/kv-compression-design.md section 9, steps 4 and 6), over the
 * committed + pending rows of `layer`; the reference has not implemented
 * them yet.
 * attention_logits: logits[(b * num_heads + h) * ld + t] = the inner-product
 * estimate <decode(q_h), decode(k_t)> (+ the QJL correction) of query head h
 * with row t of its kv head, for t < the sequence's rows; q as in
 * sai_tqcache_attend; unscaled. ld >= the longest sequence. */
sai_status sai_tqcache_attention_logits(sai_ctx* ctx, sai_tqcache* cache, int32_t layer,
                                        const void* q, int32_t dtype, int32_t batch,
                                        int32_t num_heads, float* logits, int32_t ld,
                                        void* stream);
/* weighted_value_sum: out[b, h, :] = sum_t weights[(b * num_heads + h) * ld
 * + t] * decode(v_t) over the sequence's rows (not normalised); weights and
 * out device f32 (out [batch, 1, num_heads * head_dim]). */
sai_status sai_tqcache_weighted_value_sum(sai_ctx* ctx, sai_tqcache* cache, int32_t layer,
                                          const float* weights, int32_t ld, int32_t batch,
                                          int32_t num_heads, float* out, void* stream);

/* ---- tuning / introspection ------------------------------------------------- */
/* Tokens per split-K work item of the decode kernel (0 = automatic, else a
 * multiple of 64). Returns the previous value. */
int32_t sai_set_decode_split(sai_ctx* ctx, int32_t tokens);
/* TurboQuant attention split in positions (a multiple of 256, 0 = automatic);
 * returns the previous value. Tuning only. */
int32_t sai_set_tq_split(sai_ctx* ctx, int32_t rows);
/* Waves per decode workgroup: 4 or 8, or 0 = automatic (4 for an int8
 * cache, 8 for int4). Returns the previous value. */
int32_t sai_set_decode_waves(sai_ctx* ctx, int32_t waves);
/* Split merge of the decode kernels (int8 and int4 caches): 0 = separate
 * combine kernel, 1 = the last workgroup of a (sequence, kv head) merges
 * in-kernel (the partials are handed over with agent-scope stores and loads,
 * one ticket counter per (sequence, kv head)), 2 = automatic (the default:
 * in-kernel when every sequence of the launch has the same split count, else
 * the combine kernel). Returns the previous value; other values are
 * ignored. */
int32_t sai_set_decode_merge(sai_ctx* ctx, int32_t in_kernel);
/* Tile order of the int8 decode kernel and the TurboQuant attention. Fixed:
 * each wave of a workgroup takes tiles w, w + waves, ..., so repeated calls on
 * the same inputs give bit-identical outputs (the int4 decode always does).
 * Run time: tiles are handed out from a workgroup counter, which balances the
 * waves; outputs then vary between calls within rounding. mode 1: fixed in
 * both; 0: run time in both; 2 (the default): fixed in the int8 decode
 * (~0.5 % slower at the Llama-3-8B layer shape), run time in the TurboQuant
 * attention (fixed is 6-10 % slower there). Returns the previous mode; other
 * values are ignored. No counterpart in the reference (its path is
 * deterministic). */
int32_t sai_set_decode_reproducible(sai_ctx* ctx, int32_t mode);
/* Number of workgroups and split size of the last decode launch on ctx. */
sai_status sai_last_decode_shape(const sai_ctx* ctx, int32_t* workgroups, int32_t* split_tokens);
/* Kernel launches of the last decode call on ctx: 1 (the decode kernel,
 * splits merged in-kernel or a single split) or 2 (the combine kernel
 * after it); 0 before any. */
int32_t sai_last_decode_launches(const sai_ctx* ctx);
/* Kernel timing of the decode step: with slots > 0, every sai_gqa_decode /
 * sai_gqa_with_cache call records two HIP events on its stream around the
 * decode kernel alone (not a combine kernel that follows it; an in-kernel
 * merge is part of the decode kernel), in a ring of
 * `slots` event pairs (at most 4096), so back-to-back calls are timed without
 * synchronizing between them. 0 turns timing off. Returns the previous slot
 * count. */
int32_t sai_set_decode_timing(sai_ctx* ctx, int32_t slots);
/* Decode-kernel durations in microseconds of the most recent timed calls,
 * oldest first, at most max_n of them (and at most the slot count); waits for
 * the last call's end event. Returns how many were written, or a negative
 * status. */
int32_t sai_decode_kernel_times(sai_ctx* ctx, float* us, int32_t max_n);

#ifdef __cplusplus
}
#endif

#endif /* SAI_HIP_H */
