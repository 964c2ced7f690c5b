// C++ host side of the GroupQueryAttention path over libsai_hip's C ABI.
//
// This mirrors the reference's GPU dispatch interface for the path, name for
// name, so that a caller written against it finds the same objects, argument
// meanings and error behaviour:
//
//   reference (onnx-rt/src/cuda/...)            here (namespace sai::rocm)
//   CudaRuntime::init / supports_op (mod.rs:619, :874)   RocmRuntime
//   CudaError (mod.rs:51-76, Display :78-110)            HipError
//   OpError (onnx-rt/src/operators.rs:26-49)             OpError
//   DeviceTensor (gpu_executor.rs:55-140)                DeviceTensor
//   LayerKind / KvView (kv_cache.rs:53-89)               LayerKind / KvView
//   GpuKvCache (kv_cache.rs:111-390)                     GpuKvCache
//   KvCacheDispatchCtx (gpu_executor.rs:277-280)         KvCacheDispatchCtx
//   AttributeProto (onnx_types.rs:20-95)                 AttributeProto
//   parse_gqa_attrs (gpu_executor.rs:862-884)            parse_gqa_attrs
//   gqa_validate (ops/microsoft.rs:933-984)              gqa_validate
//   dispatch_gqa (gpu_executor.rs:944-970)               dispatch_gqa
//   dispatch_rotary_embedding (gpu_executor.rs:815-851)  dispatch_rotary_embedding
//     with rotary_gpu (kernels/rotary.rs:274-374)
//   op_rotary_embedding (ops/microsoft.rs:556-652)       op_rotary_embedding
//   op_group_query_attention (ops/microsoft.rs:1082)     op_group_query_attention
//   op_multi_head_attention (ops/microsoft.rs:806)       op_multi_head_attention
//   precompute_rope_tables (model_loader/gemma.rs:458)   precompute_rope_tables
//
// Differences by design, each forced by the quantised paged cache:
//   * the cache stores int8 (per token-head scale) or int4 (group-32 scale and
//     zero) codes in 16-token pages, not bf16 rows; GpuKvCache::allocate takes
//     a KvQuant where the reference takes a storage DataType, and KvView
//     describes a paged pool instead of two linear K/V buffers;
//   * a cache holds up to max_batch sequences (the reference: batch 1);
//   * dispatch_gqa routes rank-3 [B, S, H*D] inputs through the cache (the
//     reference bypasses it for rank-3, gpu_executor.rs:886-915) and accepts
//     S > 1 (a prefill chunk: append S tokens, then attend causally);
//   * RoPE is fused: cos/sin caches at inputs 7 and 8 rotate Q and the new K
//     inside the kernels, as op_group_query_attention does on the CPU
//     (ops/microsoft.rs:1108-1133);
//   * the attention output is always f32;
//   * dispatch_rotary_embedding reads bf16 cos/sin tables directly (their
//     exact f32 values, which the reference's bf16->f32 cast produces) instead
//     of casting them into a new device tensor; op_rotary_embedding takes
//     device tensors and reads position_ids back to the host.
//
// Errors never throw: every fallible call returns Result<T, E>.
#ifndef SAI_GQA_HOST_HPP
#define SAI_GQA_HOST_HPP

#include <cstddef>
#include <cstdint>
#include <optional>
#include <string>
#include <string_view>
#include <utility>
#include <variant>
#include <vector>

#include "sai_hip.h"

namespace sai::rocm {

// ---------------------------------------------------------------- results ---
struct Unit {};

template <class T, class E>
class [[nodiscard]] Result {
 public:
  Result(T v) : v_(std::in_place_index<0>, std::move(v)) {}
  Result(E e) : v_(std::in_place_index<1>, std::move(e)) {}
  bool ok() const { return v_.index() == 0; }
  explicit operator bool() const { return ok(); }
  T& value() & { return std::get<0>(v_); }
  const T& value() const& { return std::get<0>(v_); }
  T&& value() && { return std::get<0>(std::move(v_)); }
  const E& error() const { return std::get<1>(v_); }

 private:
  std::variant<T, E> v_;
};

// ------------------------------------------------------------ error types ---
// Counterpart of CudaError (onnx-rt/src/cuda/mod.rs:51-76). to_string() follows
// its Display (mod.rs:78-110) with "HIP" in place of "CUDA".
struct HipError {
  enum class Kind { NoDevice, AllocFailed, CopyFailed, RuntimeError };
  Kind kind = Kind::RuntimeError;
  std::string op;    // RuntimeError: the failing operation; CopyFailed: the copy
  int32_t code = -1; // hipError_t or sai_status
  size_t size = 0;   // AllocFailed: requested bytes

  static HipError runtime(std::string op, int32_t code = -1);
  static HipError alloc_failed(size_t size, int32_t code);
  static HipError copy_failed(std::string what, int32_t code);
  static HipError no_device();
  std::string to_string() const;
};

// Counterpart of OpError (onnx-rt/src/operators.rs:26-37); to_string() is its
// Display (operators.rs:39-49).
struct OpError {
  enum class Kind { UnsupportedOp, ShapeMismatch, InvalidAttribute, InternalError };
  Kind kind = Kind::InternalError;
  std::string message;

  static OpError unsupported(std::string m) { return {Kind::UnsupportedOp, std::move(m)}; }
  static OpError shape(std::string m) { return {Kind::ShapeMismatch, std::move(m)}; }
  static OpError attribute(std::string m) { return {Kind::InvalidAttribute, std::move(m)}; }
  static OpError internal(std::string m) { return {Kind::InternalError, std::move(m)}; }
  std::string to_string() const;
};

// ---------------------------------------------------------------- runtime ---
// ONNX TensorProto element types (onnx-rt/src/tensor.rs DataType numbering).
enum class DataType : int32_t {
  Undefined = 0,
  Float = 1,
  UInt8 = 2,
  Int8 = 3,
  UInt16 = 4,
  Int32 = 6,
  Int64 = 7,
  Float16 = 10,
  BFloat16 = 16,
};
size_t element_size(DataType dt);
const char* data_type_name(DataType dt);

// Owns one sai_ctx (device, decode workspace, last error). Move-only.
// Replaces CudaRuntime (onnx-rt/src/cuda/mod.rs:619-700).
class RocmRuntime {
 public:
  // sai_init on `device`. NoDevice when no HIP device is visible,
  // RuntimeError{"rocm_runtime_init:not_gfx950"} when the device is not gfx950.
  static Result<RocmRuntime, HipError> init(int device = 0);
  // The ops this runtime dispatches (CudaRuntime::supports_op, mod.rs:874-889,
  // narrowed to the ops this library implements).
  static bool supports_op(std::string_view op_type);

  RocmRuntime(RocmRuntime&& o) noexcept : ctx_(std::exchange(o.ctx_, nullptr)), device_(o.device_) {}
  RocmRuntime& operator=(RocmRuntime&& o) noexcept;
  RocmRuntime(const RocmRuntime&) = delete;
  RocmRuntime& operator=(const RocmRuntime&) = delete;
  ~RocmRuntime();

  int device() const { return device_; }
  sai_ctx* raw() const { return ctx_; }
  // Blocks until all work on the device is done.
  Result<Unit, HipError> synchronize() const;
  // The C ABI's message for the last failed call on this runtime.
  std::string last_error() const;

 private:
  RocmRuntime(sai_ctx* c, int device) : ctx_(c), device_(device) {}
  sai_ctx* ctx_ = nullptr;
  int device_ = 0;
};

// Device allocation (hipMalloc / hipFree). Move-only; may be empty.
class DeviceBuffer {
 public:
  DeviceBuffer() = default;
  static Result<DeviceBuffer, HipError> alloc(size_t bytes);
  DeviceBuffer(DeviceBuffer&& o) noexcept
      : ptr_(std::exchange(o.ptr_, nullptr)), bytes_(std::exchange(o.bytes_, 0)) {}
  DeviceBuffer& operator=(DeviceBuffer&& o) noexcept;
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  ~DeviceBuffer();

  void* as_ptr() const { return ptr_; }
  size_t size() const { return bytes_; }
  Result<Unit, HipError> copy_from_host(const void* src, size_t bytes);
  Result<Unit, HipError> copy_to_host(void* dst, size_t bytes) const;

 private:
  void* ptr_ = nullptr;
  size_t bytes_ = 0;
};

// A typed, shaped device tensor (gpu_executor.rs:55-140).
struct DeviceTensor {
  DeviceBuffer buffer;
  std::vector<int64_t> shape;
  DataType dtype = DataType::Float;
  std::string name;

  size_t total_elements() const;  // 0 when any dim is negative
  size_t byte_size() const;
  // The buffer holds at least byte_size() bytes (and a device pointer when
  // that is not 0): shape and buffer are separate fields, and every entry
  // point checks this before a kernel reads or writes the tensor.
  bool holds_shape() const;
  // Uninitialised device tensor of `shape` and `dtype`.
  static Result<DeviceTensor, HipError> alloc(std::vector<int64_t> shape, DataType dtype);
  // Device copy of little-endian host bytes (Tensor::raw_data). The byte
  // count must equal the shape's byte size.
  static Result<DeviceTensor, HipError> from_host(const void* raw, size_t bytes,
                                                  std::vector<int64_t> shape, DataType dtype,
                                                  std::string name = {});
  static Result<DeviceTensor, HipError> from_f32(const std::vector<float>& v,
                                                 std::vector<int64_t> shape);
  Result<std::vector<uint8_t>, HipError> to_host() const;
  // f32 tensors only (RuntimeError{"to_host_f32:dtype"} otherwise).
  Result<std::vector<float>, HipError> to_host_f32() const;
};

// ------------------------------------------------------------------ cache ---
// kv_cache.rs:53-57. A sliding-window layer's queries see their last `window`
// keys (the pages keep every token); window 0 is rejected at allocation.
struct LayerKind {
  enum class Tag { Global, SlidingWindow };
  Tag tag = Tag::Global;
  size_t window = 0;
  static LayerKind global() { return {Tag::Global, 0}; }
  static LayerKind sliding_window(size_t w) { return {Tag::SlidingWindow, w}; }
  bool operator==(const LayerKind& o) const { return tag == o.tag && window == o.window; }
};

enum class KvQuant : int32_t { Int8 = SAI_KV_INT8, Int4 = SAI_KV_INT4 };

// The reference's KvView (kv_cache.rs:72-80) points at linear K and V rows;
// here one pool per layer holds both, in (page, kv head) blocks of
// block_bytes (K codes, V codes, then the quantisation parameters). Tokens
// [start_token, start_token + token_count) of every sequence are in view
// (start_token > 0 only for a sliding-window layer, kv_cache.rs:351-358).
struct KvView {
  const void* pool = nullptr;
  size_t pool_bytes = 0;
  size_t block_bytes = 0;
  size_t start_token = 0;
  size_t token_count = 0;
  size_t num_kv_heads = 0;
  size_t head_dim = 0;
  size_t batch = 0;
  KvQuant quant = KvQuant::Int8;
};

// RoPE tables for a fused append: device f32 [rows, head_dim/2].
struct RopeTables {
  const float* cos = nullptr;
  const float* sin = nullptr;
  int32_t rows = 0;
  bool interleaved = false;
};

// Per-layer quantised paged KV cache (kv_cache.rs:111-390) with the
// reference's lifecycle: append leaves the step's tokens pending, attention
// sees committed + pending tokens (view_pending), advance_position commits
// them once per forward pass. Move-only.
class GpuKvCache {
 public:
  // kv_cache.rs:129-203. Every sequence slot b in [0, max_batch) owns
  // ceil(max_seq_len / 16) pages of its own (identity page table); the pools
  // are zero-filled. Errors: RuntimeError "kv_cache_allocate:layer_kinds_len",
  // "kv_cache_allocate:zero_dim", "kv_cache_allocate:sliding_window" (window
  // 0 or above i32), "kv_cache_allocate:unsupported_head_dim"; AllocFailed.
  static Result<GpuKvCache, HipError> allocate(RocmRuntime& rt, size_t num_layers,
                                               size_t num_kv_heads, size_t head_dim,
                                               size_t max_seq_len, KvQuant quant,
                                               const std::vector<LayerKind>& layer_kinds,
                                               size_t max_batch = 1);
  GpuKvCache(GpuKvCache&& o) noexcept;
  GpuKvCache& operator=(GpuKvCache&& o) noexcept;
  GpuKvCache(const GpuKvCache&) = delete;
  GpuKvCache& operator=(const GpuKvCache&) = delete;
  ~GpuKvCache();

  size_t num_layers() const { return num_layers_; }
  size_t num_kv_heads() const { return num_kv_heads_; }
  size_t head_dim() const { return head_dim_; }
  size_t max_seq_len() const { return max_seq_len_; }
  size_t max_batch() const { return max_batch_; }
  KvQuant quant() const { return quant_; }
  // Committed tokens per sequence (every sequence advances together).
  size_t current_position() const { return position_; }
  // Tokens appended in this forward pass and not yet committed.
  size_t pending() const;
  // Sequences of the current pass (set by the first append at position 0).
  size_t batch() const { return batch_; }

  // kv_cache.rs:233-278: write the pass's new K/V for one layer. new_k,
  // new_v: [B, S, Hkv*D] (rank 3) or [B, Hkv, 1, D] (rank 4, S = 1), Float or
  // BFloat16, pre-RoPE when `rope` is given. Errors: RuntimeError
  // "kv_cache_append:layer_idx", ":position_overflow",
  // ":tensor_byte_size_mismatch", ":dtype_mismatch", ":batch_mismatch",
  // ":pending_mismatch" (another layer of this pass appended a different S).
  Result<Unit, HipError> append(size_t layer_idx, const DeviceTensor& new_k,
                                const DeviceTensor& new_v, const RopeTables* rope = nullptr,
                                void* stream = nullptr);
  // The checks append() makes before writing (sequence count, capacity,
  // pending count of this pass), for a caller that writes the tokens through
  // the fused decode kernel instead; switches the batch at position 0.
  Result<Unit, HipError> check_append(size_t batch, size_t s_new);
  // kv_cache.rs:295-304: commit the pending tokens. Errors: RuntimeError
  // "kv_cache_advance:position_overflow", "kv_cache_advance:nothing_pending".
  Result<Unit, HipError> advance_position(void* stream = nullptr);
  // kv_cache.rs:300-390: committed tokens, and committed + pending (the last
  // `window` of them for a sliding-window layer).
  Result<KvView, HipError> view(size_t layer_idx) const;
  Result<KvView, HipError> view_pending(size_t layer_idx) const;
  // kv_cache.rs:386-388: position back to 0, buffers kept.
  void reset();

  // Dequantised copy (host, f32) of tokens [t0, t0+n) of one (sequence,
  // kv head) of a layer: k and v are [n][head_dim]. Synchronous.
  Result<std::pair<std::vector<float>, std::vector<float>>, HipError> read_dequantized(
      size_t layer_idx, size_t seq, size_t kv_head, size_t t0, size_t n) const;

  sai_kvcache* raw() const { return cache_; }
  RocmRuntime& runtime() const { return *rt_; }

 private:
  GpuKvCache() = default;
  Result<Unit, HipError> ensure_batch(size_t batch, const char* op);
  Result<KvView, HipError> view_at(size_t layer_idx, size_t count, const char* op) const;

  RocmRuntime* rt_ = nullptr;
  sai_kvcache* cache_ = nullptr;
  size_t num_layers_ = 0, num_kv_heads_ = 0, head_dim_ = 0, max_seq_len_ = 0, max_batch_ = 0;
  size_t pages_per_seq_ = 0;
  std::vector<size_t> layer_windows_;  // 0: global
  size_t batch_ = 0;
  size_t position_ = 0;
  KvQuant quant_ = KvQuant::Int8;
};

// gpu_executor.rs:277-280: the cache plus the layer the next GQA node uses.
struct KvCacheDispatchCtx {
  GpuKvCache* cache = nullptr;
  size_t next_layer_idx = 0;
};

// ------------------------------------------------------------- operator ---
// onnx_types.rs:20-95, the fields this op reads.
enum class AttributeType : int32_t { Undefined = 0, Float = 1, Int = 2, String = 3 };
struct AttributeProto {
  std::string name;
  AttributeType attr_type = AttributeType::Undefined;
  float f = 0.0f;
  int64_t i = 0;
  std::string s;
  static AttributeProto make_int(std::string n, int64_t v);
  static AttributeProto make_float(std::string n, float v);
};

// Attributes of com.microsoft.GroupQueryAttention with the defaults of
// dispatch_microsoft_fused (executor.rs:2341-2361): num_heads = kv_num_heads = 0,
// local_window_size = -1, do_rotary = 1, rotary_interleaved = 0, scale unset.
// do_rotary_set records whether the node carried the attribute at all.
struct GqaAttrs {
  int64_t num_heads = 0;
  int64_t kv_num_heads = 0;
  int64_t local_window_size = -1;
  bool do_rotary = true;
  bool do_rotary_set = false;
  bool rotary_interleaved = false;
  std::optional<float> scale;
};
GqaAttrs parse_gqa_attrs(const std::vector<AttributeProto>& attrs);

// Shape facts gqa_validate derives (ops/microsoft.rs:933-984).
struct GqaShape {
  size_t num_heads = 0, kv_heads = 0, batch = 0, seq = 0, q_hidden = 0, head_dim = 0;
};
// ops/microsoft.rs:933-984 for rank-3 Q/K/V, same checks and messages.
// Rank-4 [B, H, 1, D] Q/K/V (the reference's cache path, attention.rs:1268-1281)
// take their head counts from the shapes.
Result<GqaShape, OpError> gqa_validate(const std::vector<int64_t>& q_shape,
                                       const std::vector<int64_t>& k_shape,
                                       const std::vector<int64_t>& v_shape, int64_t num_heads,
                                       int64_t kv_num_heads);

// gpu_executor.rs:944-970. Inputs by slot: 0 query, 1 key, 2 value, 3/4
// past_key/past_value (unused: the cache holds the past), 5/6 seqlens_k /
// total_sequence_length (advisory, unused as on the CPU), 7 cos_cache,
// 8 sin_cache. Returns { attn_out [B, S, Hq*D] } in Q's dtype (f32, or bf16
// rounded to nearest even, as gpu_gqa returns, attention.rs:835, :877-901);
// present K/V stay in the cache. With kv_cache_ctx, the node uses layer next_layer_idx (then
// incremented, also on error, as in the reference); S = 1 runs the fused
// append + split-K decode, S > 1 appends S tokens then runs the prefill
// kernel. Without kv_cache_ctx the node attends over its own K/V only
// through a transient one-layer cache. RoPE: applied when cos/sin are given
// and do_rotary is 1; an explicit do_rotary=1 without them is the CPU op's
// ShapeMismatch. local_window_size > 0 limits each query at position p to
// keys [p - local_window_size, p] (the GPU mask, attention.rs:79), on top of
// a sliding-window cache layer's last-w-keys rule; other values mean no
// window (gpu_executor.rs:874-878). Asynchronous on the null stream.
Result<std::vector<DeviceTensor>, OpError> dispatch_gqa(
    RocmRuntime& runtime, const std::vector<const DeviceTensor*>& inputs,
    const std::vector<AttributeProto>& attrs, KvCacheDispatchCtx* kv_cache_ctx);

// Outputs of the CPU attention ops: attention [B, S, Hq*D] f32 and present
// K/V [B, Hkv, past + S, D] f32.
struct AttentionOutputs {
  DeviceTensor attn, present_key, present_value;
};

// ops/microsoft.rs:1082-1190 (op_group_query_attention) on device tensors,
// with its checks, order and messages: Float Q/K/V [B, S, H*D], optional
// past_key / past_value [B, Hkv, P, D] at inputs 3/4, cos/sin at 7/8 when
// do_rotary, local_window_size must be -1. present_key = past ++ RoPE(new K)
// and present_value = past ++ new V, copied exactly (sai_copy_rows,
// sai_rotary_embedding); the attention runs over a transient int8 paged
// cache holding them (outputs within the kernels' tolerance). head_dim 64 or
// 128 and a group of 1, 2, 4 or 8 (else UnsupportedOp).
Result<AttentionOutputs, OpError> op_group_query_attention(
    RocmRuntime& runtime, const std::vector<const DeviceTensor*>& inputs, int64_t num_heads,
    int64_t kv_num_heads, std::optional<float> scale_attr, int64_t local_window_size,
    bool do_rotary, bool rotary_interleaved);

// ops/microsoft.rs:806-925 (op_multi_head_attention): Q/K/V [B, S, H*D] of
// one shape, optional past_key / past_value at inputs 6/7, no RoPE, causal
// over past + new; the same present outputs and attention path as above.
Result<AttentionOutputs, OpError> op_multi_head_attention(
    RocmRuntime& runtime, const std::vector<const DeviceTensor*>& inputs, int64_t num_heads,
    std::optional<float> scale_attr);

// gpu_executor.rs:815-851 over rotary_gpu (kernels/rotary.rs:274-374).
// Inputs: [X, position_ids, cos_cache, sin_cache] (4 or more) or
// [X, cos_cache, sin_cache]. The start position is the first i64 of
// position_ids (its first 8 bytes, truncated to i32; 0 when it holds fewer
// than 8 bytes), else the cache's current_position(), else 0; row s of every
// sequence uses table row start + s. X: [B, H, S, D] or [B, S, H*D] (rank 3:
// num_heads from the attribute, else hidden / (2 * table inner dim)), Float or
// BFloat16; tables Float or BFloat16 [max_seq, D/2]; attribute `interleaved`.
// Returns { Y } of X's shape and dtype. Errors: InternalError
// "GPU RotaryEmbedding: missing input '...'", and "ROCm RotaryEmbedding: "
// followed by the HipError of rotary_gpu's checks (same wording).
// Asynchronous on the null stream, except the position_ids read-back.
Result<std::vector<DeviceTensor>, OpError> dispatch_rotary_embedding(
    RocmRuntime& runtime, const std::vector<const DeviceTensor*>& inputs,
    const std::vector<AttributeProto>& attrs, const KvCacheDispatchCtx* kv_cache_ctx);

// ops/microsoft.rs:556-652 on device tensors, with the CPU op's checks, order
// and messages: Float X of rank 4 [B, H, S, D], or rank 3 [B, S, H*D] read as
// [B, num_heads, S, D] without a transpose; position_ids Int64 or Int32 of
// S or B*S entries (read back to the host and range-checked); rotary_dim
// <= 0 means D, else a partial rotation with the tail copied. Returns Y (Float,
// X's shape).
Result<DeviceTensor, OpError> op_rotary_embedding(RocmRuntime& runtime,
                                                  const std::vector<const DeviceTensor*>& inputs,
                                                  bool interleaved, int64_t rotary_embedding_dim,
                                                  int64_t num_heads_attr);

// model_loader/gemma.rs:458-472: (cos, sin) BFloat16 device tensors
// [max_pos, half], bit for bit the loader's tables. Errors: RuntimeError
// "precompute_rope_tables" with the C ABI status; AllocFailed.
Result<std::pair<DeviceTensor, DeviceTensor>, HipError> precompute_rope_tables(
    RocmRuntime& runtime, size_t max_pos, size_t half, float rope_theta);

}  // namespace sai::rocm

#endif  // SAI_GQA_HOST_HPP
