// GpuCompressedKvCache: CompressedKVCache (onnx-rt/src/kv_compression.rs:
// 738-963) over the sai_tqcache_* C ABI.
#include "kv_compression.hpp"

#include <algorithm>
#include <limits>
#include <string>

namespace sai::rocm {
namespace {

OpError op_error(sai_status st, const std::string& prefix, const RocmRuntime& rt) {
  OpError::Kind k = OpError::Kind::InternalError;
  switch (st) {
    case SAI_ERR_UNSUPPORTED: k = OpError::Kind::UnsupportedOp; break;
    case SAI_ERR_INVALID_ATTRIBUTE: k = OpError::Kind::InvalidAttribute; break;
    case SAI_ERR_SHAPE_MISMATCH:
    case SAI_ERR_OVERFLOW: k = OpError::Kind::ShapeMismatch; break;
    default: break;
  }
  return OpError{k, prefix + rt.last_error()};
}

// sai dtype of a K/V/Q tensor: Float or BFloat16 only.
std::optional<int32_t> row_dtype(const DeviceTensor& t) {
  if (t.dtype == DataType::Float) return SAI_DTYPE_F32;
  if (t.dtype == DataType::BFloat16) return SAI_DTYPE_BF16;
  return std::nullopt;
}

bool fits_i32(size_t v) { return v <= (size_t)std::numeric_limits<int32_t>::max(); }

}  // namespace

Result<GpuCompressedKvCache, OpError> GpuCompressedKvCache::create(RocmRuntime& rt,
                                                                   const KVCacheConfig& cfg,
                                                                   size_t max_batch,
                                                                   size_t max_rows) {
  const std::string pre = "CompressedKVCache: ";
  if (!fits_i32(cfg.num_layers) || !fits_i32(cfg.num_kv_heads) || !fits_i32(cfg.head_dim) ||
      !fits_i32(max_batch) || !fits_i32(max_rows))
    return OpError::shape(pre + "sizes beyond i32");
  sai_tqcache_desc d{};
  d.num_layers = (int32_t)cfg.num_layers;
  d.num_kv_heads = (int32_t)cfg.num_kv_heads;
  d.head_dim = (int32_t)cfg.head_dim;
  d.bits = cfg.kv_quant_bits;
  d.qjl = cfg.kv_qjl_residual ? 1 : 0;
  d.max_batch = (int32_t)max_batch;
  d.max_rows = (int32_t)max_rows;
  d.seed = cfg.seed;
  d.lowrank_k =
      cfg.kv_lowrank_k ? (int32_t)std::min<size_t>(std::max<size_t>(*cfg.kv_lowrank_k, 1), 1u << 30)
                       : 0;
  GpuCompressedKvCache c;
  c.rt_ = &rt;
  const sai_status st = sai_tqcache_create(rt.raw(), &d, &c.cache_);
  if (st != SAI_OK) return op_error(st, pre, rt);
  c.cfg_ = cfg;
  c.max_batch_ = max_batch;
  c.max_rows_ = max_rows;
  return c;
}

GpuCompressedKvCache::GpuCompressedKvCache(GpuCompressedKvCache&& o) noexcept
    : rt_(o.rt_), cache_(std::exchange(o.cache_, nullptr)), cfg_(o.cfg_),
      max_batch_(o.max_batch_), max_rows_(o.max_rows_) {}

GpuCompressedKvCache& GpuCompressedKvCache::operator=(GpuCompressedKvCache&& o) noexcept {
  if (this != &o) {
    if (cache_) sai_tqcache_destroy(cache_);
    rt_ = o.rt_;
    cache_ = std::exchange(o.cache_, nullptr);
    cfg_ = o.cfg_;
    max_batch_ = o.max_batch_;
    max_rows_ = o.max_rows_;
  }
  return *this;
}

GpuCompressedKvCache::~GpuCompressedKvCache() {
  if (cache_) sai_tqcache_destroy(cache_);
}

Result<Unit, OpError> GpuCompressedKvCache::write_kv(size_t layer, const DeviceTensor& k,
                                                     const DeviceTensor& v, void* stream) {
  const std::string pre = "CompressedKVCache::write_kv: ";
  const auto dt = row_dtype(k);
  if (!dt || k.dtype != v.dtype) return OpError::unsupported(pre + "K/V must be Float or BFloat16 alike");
  const int64_t hidden = (int64_t)(cfg_.num_kv_heads * cfg_.head_dim);
  if (k.shape.size() != 3 || k.shape != v.shape || k.shape[2] != hidden || k.shape[0] <= 0 ||
      k.shape[1] <= 0 || !fits_i32((size_t)k.shape[0]) || !fits_i32((size_t)k.shape[1]) ||
      !fits_i32(layer))
    return OpError::shape(pre + "K/V must be [batch, rows, kv_heads * head_dim]");
  if (!k.holds_shape() || !v.holds_shape())
    return OpError::shape(pre + "K/V buffer does not hold its shape");
  const sai_status st =
      sai_tqcache_write(rt_->raw(), cache_, (int32_t)layer, k.buffer.as_ptr(), v.buffer.as_ptr(),
                        *dt, (int32_t)k.shape[0], (int32_t)k.shape[1], stream);
  if (st != SAI_OK) return op_error(st, pre, *rt_);
  return Unit{};
}

Result<Unit, OpError> GpuCompressedKvCache::advance(void* stream) {
  const sai_status st = sai_tqcache_advance(rt_->raw(), cache_, stream);
  if (st != SAI_OK) return op_error(st, "CompressedKVCache::advance: ", *rt_);
  return Unit{};
}

Result<Unit, OpError> GpuCompressedKvCache::reset() {
  const sai_status st = sai_tqcache_reset(rt_->raw(), cache_);
  if (st != SAI_OK) return op_error(st, "CompressedKVCache::reset: ", *rt_);
  return Unit{};
}

Result<Unit, OpError> GpuCompressedKvCache::read(size_t layer, size_t seq, size_t head,
                                                 size_t start, size_t len, std::vector<float>* k,
                                                 std::vector<float>* v) const {
  const std::string pre = "CompressedKVCache::read: ";
  if (!fits_i32(layer) || !fits_i32(seq) || !fits_i32(head) || !fits_i32(start) ||
      !fits_i32(len))
    return OpError::shape(pre + "index beyond i32");
  std::vector<float> kk(len * cfg_.head_dim), vv(len * cfg_.head_dim);
  const sai_status st = sai_tqcache_read(rt_->raw(), cache_, (int32_t)layer, (int32_t)seq,
                                         (int32_t)head, (int32_t)start, (int32_t)len, kk.data(),
                                         vv.data());
  if (st != SAI_OK) return op_error(st, pre, *rt_);
  if (k) *k = std::move(kk);
  if (v) *v = std::move(vv);
  return Unit{};
}

Result<std::vector<float>, OpError> GpuCompressedKvCache::read_k(size_t layer, size_t seq,
                                                                 size_t head, size_t start,
                                                                 size_t len) const {
  std::vector<float> k;
  auto r = read(layer, seq, head, start, len, &k, nullptr);
  if (!r) return r.error();
  return k;
}

Result<std::vector<float>, OpError> GpuCompressedKvCache::read_v(size_t layer, size_t seq,
                                                                 size_t head, size_t start,
                                                                 size_t len) const {
  std::vector<float> v;
  auto r = read(layer, seq, head, start, len, nullptr, &v);
  if (!r) return r.error();
  return v;
}

size_t GpuCompressedKvCache::memory_bytes() const {
  uint64_t r = 0;
  (void)sai_tqcache_memory_bytes(cache_, &r, nullptr);
  return (size_t)r;
}

size_t GpuCompressedKvCache::seq_len(size_t seq) const {
  std::vector<int32_t> lens(max_batch_);
  if (seq >= max_batch_ || sai_tqcache_lengths(cache_, lens.data(), nullptr, nullptr) != SAI_OK)
    return 0;
  return (size_t)lens[seq];
}

Result<DeviceTensor, OpError> GpuCompressedKvCache::attend(size_t layer, const DeviceTensor& q,
                                                           size_t num_heads,
                                                           std::optional<float> scale,
                                                           void* stream) {
  const std::string pre = "CompressedKVCache::attend: ";
  const auto dt = row_dtype(q);
  if (!dt) return OpError::unsupported(pre + "query must be Float or BFloat16");
  if (q.shape.size() != 3 || q.shape[1] != 1 || q.shape[0] <= 0 || !fits_i32((size_t)q.shape[0]) ||
      !fits_i32(num_heads) || !fits_i32(layer) ||
      q.shape[2] != (int64_t)(num_heads * cfg_.head_dim))
    return OpError::shape(pre + "query must be [batch, 1, num_heads * head_dim]");
  if (!q.holds_shape()) return OpError::shape(pre + "query buffer does not hold its shape");
  auto out = DeviceTensor::alloc(q.shape, DataType::Float);
  if (!out) return OpError::internal(pre + out.error().to_string());
  const sai_status st = sai_tqcache_attend(rt_->raw(), cache_, (int32_t)layer, q.buffer.as_ptr(),
                                           *dt, (int32_t)q.shape[0], (int32_t)num_heads,
                                           scale ? 1 : 0, scale.value_or(0.0f),
                                           (float*)out.value().buffer.as_ptr(), stream);
  if (st != SAI_OK) return op_error(st, pre, *rt_);
  return std::move(out).value();
}

Result<DeviceTensor, OpError> GpuCompressedKvCache::write_attend(
    size_t layer, const DeviceTensor& q, const DeviceTensor& k_new, const DeviceTensor& v_new,
    size_t num_heads, std::optional<float> scale, void* stream) {
  const std::string pre = "CompressedKVCache::write_attend: ";
  const auto qd = row_dtype(q), kd = row_dtype(k_new);
  if (!qd || !kd || k_new.dtype != v_new.dtype)
    return OpError::unsupported(pre + "Q and K/V must be Float or BFloat16");
  const int64_t hidden = (int64_t)(cfg_.num_kv_heads * cfg_.head_dim);
  if (q.shape.size() != 3 || q.shape[1] != 1 || q.shape[0] <= 0 || !fits_i32((size_t)q.shape[0]) ||
      !fits_i32(num_heads) || !fits_i32(layer) ||
      q.shape[2] != (int64_t)(num_heads * cfg_.head_dim) || k_new.shape != v_new.shape ||
      k_new.shape != std::vector<int64_t>{q.shape[0], 1, hidden})
    return OpError::shape(pre + "Q [batch, 1, Hq*D] and K/V [batch, 1, Hkv*D] expected");
  if (!q.holds_shape() || !k_new.holds_shape() || !v_new.holds_shape())
    return OpError::shape(pre + "Q/K/V buffer does not hold its shape");
  auto out = DeviceTensor::alloc(q.shape, DataType::Float);
  if (!out) return OpError::internal(pre + out.error().to_string());
  const sai_status st = sai_tqcache_write_attend(
      rt_->raw(), cache_, (int32_t)layer, q.buffer.as_ptr(), *qd, k_new.buffer.as_ptr(),
      v_new.buffer.as_ptr(), *kd, (int32_t)q.shape[0], (int32_t)num_heads, scale ? 1 : 0,
      scale.value_or(0.0f), (float*)out.value().buffer.as_ptr(), stream);
  if (st != SAI_OK) return op_error(st, pre, *rt_);
  return std::move(out).value();
}

}  // namespace sai::rocm
