// Host side of the TurboQuant compressed KV cache: the counterpart of
// CompressedKVCache and KVCacheConfig (onnx-rt/src/kv_compression.rs:694-963)
// over the sai_tqcache_* C ABI. The reference keeps one row per
// write_kv(layer, head, pos, k, v) call in host memory; this cache lives on the
// device and takes a pass per call: every kv head of a layer for a batch of
// sequences, rows left pending until advance() (as GpuKvCache does).
#pragma once

#include <cstddef>
#include <cstdint>
#include <optional>
#include <vector>

#include "gqa_host.hpp"

namespace sai::rocm {

// KVCacheConfig (kv_compression.rs:694-727), with its defaults.
struct KVCacheConfig {
  uint8_t kv_quant_bits = 4;
  bool kv_qjl_residual = true;
  std::optional<size_t> kv_lowrank_k;  // Some(0) counts as Some(1)
  size_t num_layers = 1;
  size_t num_kv_heads = 1;
  size_t head_dim = 64;
  uint64_t seed = 0xDEADBEEFCAFE1234ull;
};

// CompressedKVCache (kv_compression.rs:738-963) on the device. Move-only.
// Errors are the op's: UnsupportedOp (head_dim other than 64, 128, 256; a
// pass the cache cannot take), InvalidAttribute ("bits must be 3, 4, or 8"),
// ShapeMismatch (indices, sizes, lengths past max_rows), InternalError.
class GpuCompressedKvCache {
 public:
  static Result<GpuCompressedKvCache, OpError> create(RocmRuntime& rt, const KVCacheConfig& cfg,
                                                     size_t max_batch, size_t max_rows);
  GpuCompressedKvCache(GpuCompressedKvCache&& o) noexcept;
  GpuCompressedKvCache& operator=(GpuCompressedKvCache&& o) noexcept;
  GpuCompressedKvCache(const GpuCompressedKvCache&) = delete;
  GpuCompressedKvCache& operator=(const GpuCompressedKvCache&) = delete;
  ~GpuCompressedKvCache();

  const KVCacheConfig& config() const { return cfg_; }

  // write_kv (:811-853) for every kv head of `layer`: k, v [B, S, Hkv*D]
  // Float or BFloat16, rows seq_len(b) .. seq_len(b) + S - 1 of sequence b.
  Result<Unit, OpError> write_kv(size_t layer, const DeviceTensor& k, const DeviceTensor& v,
                                 void* stream = nullptr);
  // Commits the pass's rows (one call per pass).
  Result<Unit, OpError> advance(void* stream = nullptr);
  // Every sequence back to 0 rows, storage kept.
  Result<Unit, OpError> reset();
  // read_k / read_v (:862-907): rows [start, start+len) of (layer, sequence,
  // kv head), [len][head_dim] f32; read_k prefers the low-rank K when kept.
  Result<std::vector<float>, OpError> read_k(size_t layer, size_t seq, size_t head, size_t start,
                                             size_t len) const;
  Result<std::vector<float>, OpError> read_v(size_t layer, size_t seq, size_t head, size_t start,
                                             size_t len) const;
  // memory_bytes (:928-957), the reference's accounting of the committed rows.
  size_t memory_bytes() const;
  // seq_len (:960-962): committed rows of a sequence (every head alike).
  size_t seq_len(size_t seq) const;

  // Decode attention of q [B, 1, Hq*D] (RoPE applied) over each sequence's
  // rows including this pass's; out [B, 1, Hq*D] f32 (allocated here).
  Result<DeviceTensor, OpError> attend(size_t layer, const DeviceTensor& q, size_t num_heads,
                                       std::optional<float> scale = {}, void* stream = nullptr);
  // write_kv of one row per sequence and attend, in one launch.
  Result<DeviceTensor, OpError> write_attend(size_t layer, const DeviceTensor& q,
                                             const DeviceTensor& k_new, const DeviceTensor& v_new,
                                             size_t num_heads, std::optional<float> scale = {},
                                             void* stream = nullptr);

  sai_tqcache* raw() const { return cache_; }

 private:
  GpuCompressedKvCache() = default;
  Result<Unit, OpError> read(size_t layer, size_t seq, size_t head, size_t start, size_t len,
                             std::vector<float>* k, std::vector<float>* v) const;

  RocmRuntime* rt_ = nullptr;
  sai_tqcache* cache_ = nullptr;
  KVCacheConfig cfg_;
  size_t max_batch_ = 0, max_rows_ = 0;
};

}  // namespace sai::rocm
