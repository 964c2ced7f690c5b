// Implementation of the C++ host side (gqa_host.hpp) over libsai_hip's C ABI.
// Host code only: device work is done by the library's kernels; this file
// validates, keeps the cache bookkeeping and maps status codes to errors.
#include "gqa_host.hpp"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <limits>

namespace sai::rocm {

namespace {

std::string fmt_code(const char* fmt, const std::string& a, long long b) {
  char buf[512];
  std::snprintf(buf, sizeof buf, fmt, a.c_str(), b);
  return buf;
}

OpError::Kind kind_of(sai_status st) {
  switch (st) {
    case SAI_ERR_INVALID_ATTRIBUTE: return OpError::Kind::InvalidAttribute;
    case SAI_ERR_SHAPE_MISMATCH: return OpError::Kind::ShapeMismatch;
    case SAI_ERR_UNSUPPORTED: return OpError::Kind::UnsupportedOp;
    default: return OpError::Kind::InternalError;
  }
}

// IEEE binary16 -> binary32, exact (every half is a float).
float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t mant = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0x1Fu) {
    bits = sign | 0x7F800000u | (mant << 13);
  } else if (exp != 0) {
    bits = sign | ((exp + 112u) << 23) | (mant << 13);
  } else if (mant == 0) {
    bits = sign;
  } else {
    // subnormal: normalise
    int e = -1;
    do {
      mant <<= 1;
      ++e;
    } while ((mant & 0x400u) == 0);
    bits = sign | ((uint32_t)(112 - e) << 23) | ((mant & 0x3FFu) << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

bool is_float_like(DataType dt) { return dt == DataType::Float || dt == DataType::BFloat16; }

int32_t sai_dtype(DataType dt) {
  return dt == DataType::BFloat16 ? SAI_DTYPE_BF16 : SAI_DTYPE_F32;
}

}  // namespace

// ----------------------------------------------------------------- errors ---
HipError HipError::runtime(std::string op, int32_t code) {
  HipError e;
  e.kind = Kind::RuntimeError;
  e.op = std::move(op);
  e.code = code;
  return e;
}
HipError HipError::alloc_failed(size_t size, int32_t code) {
  HipError e;
  e.kind = Kind::AllocFailed;
  e.size = size;
  e.code = code;
  return e;
}
HipError HipError::copy_failed(std::string what, int32_t code) {
  HipError e;
  e.kind = Kind::CopyFailed;
  e.op = std::move(what);
  e.code = code;
  return e;
}
HipError HipError::no_device() {
  HipError e;
  e.kind = Kind::NoDevice;
  return e;
}

std::string HipError::to_string() const {
  switch (kind) {
    case Kind::NoDevice: return "no HIP device found";
    case Kind::AllocFailed: {
      char buf[96];
      std::snprintf(buf, sizeof buf, "hipMalloc(%zu bytes) failed: code %d", size, code);
      return buf;
    }
    case Kind::CopyFailed: return fmt_code("hipMemcpy %s failed: code %lld", op, code);
    case Kind::RuntimeError: break;
  }
  return fmt_code("HIP %s failed: code %lld", op, code);
}

std::string OpError::to_string() const {
  switch (kind) {
    case Kind::UnsupportedOp: return "unsupported operator: " + message;
    case Kind::ShapeMismatch: return "shape mismatch: " + message;
    case Kind::InvalidAttribute: return "invalid attribute: " + message;
    case Kind::InternalError: break;
  }
  return "internal error: " + message;
}

size_t element_size(DataType dt) {
  switch (dt) {
    case DataType::Float: case DataType::Int32: return 4;
    case DataType::Int64: return 8;
    case DataType::Float16: case DataType::BFloat16: case DataType::UInt16: return 2;
    case DataType::UInt8: case DataType::Int8: return 1;
    case DataType::Undefined: break;
  }
  return 0;
}

const char* data_type_name(DataType dt) {
  switch (dt) {
    case DataType::Float: return "Float";
    case DataType::UInt8: return "UInt8";
    case DataType::Int8: return "Int8";
    case DataType::UInt16: return "UInt16";
    case DataType::Int32: return "Int32";
    case DataType::Int64: return "Int64";
    case DataType::Float16: return "Float16";
    case DataType::BFloat16: return "BFloat16";
    case DataType::Undefined: break;
  }
  return "Undefined";
}

// ---------------------------------------------------------------- runtime ---
Result<RocmRuntime, HipError> RocmRuntime::init(int device) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0 || device < 0 || device >= n)
    return HipError::no_device();
  if (!sai_device_supported(device)) return HipError::runtime("rocm_runtime_init:not_gfx950");
  sai_ctx* c = nullptr;
  const sai_status st = sai_init(device, &c);
  if (st != SAI_OK || !c) return HipError::runtime("rocm_runtime_init", st);
  return RocmRuntime(c, device);
}

bool RocmRuntime::supports_op(std::string_view op_type) {
  return op_type == "GroupQueryAttention" || op_type == "RotaryEmbedding";
}

RocmRuntime& RocmRuntime::operator=(RocmRuntime&& o) noexcept {
  if (this != &o) {
    if (ctx_) sai_destroy(ctx_);
    ctx_ = std::exchange(o.ctx_, nullptr);
    device_ = o.device_;
  }
  return *this;
}

RocmRuntime::~RocmRuntime() {
  if (ctx_) sai_destroy(ctx_);
}

Result<Unit, HipError> RocmRuntime::synchronize() const {
  if (hipSetDevice(device_) != hipSuccess) return HipError::runtime("synchronize:set_device");
  const hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return HipError::runtime("synchronize", (int32_t)e);
  return Unit{};
}

std::string RocmRuntime::last_error() const { return ctx_ ? sai_last_error(ctx_) : ""; }

// ----------------------------------------------------------- device memory ---
Result<DeviceBuffer, HipError> DeviceBuffer::alloc(size_t bytes) {
  DeviceBuffer b;
  if (bytes == 0) return b;
  const hipError_t e = hipMalloc(&b.ptr_, bytes);
  if (e != hipSuccess) {
    b.ptr_ = nullptr;
    return HipError::alloc_failed(bytes, (int32_t)e);
  }
  b.bytes_ = bytes;
  return b;
}

DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& o) noexcept {
  if (this != &o) {
    if (ptr_) (void)hipFree(ptr_);
    ptr_ = std::exchange(o.ptr_, nullptr);
    bytes_ = std::exchange(o.bytes_, 0);
  }
  return *this;
}

DeviceBuffer::~DeviceBuffer() {
  if (ptr_) (void)hipFree(ptr_);
}

Result<Unit, HipError> DeviceBuffer::copy_from_host(const void* src, size_t bytes) {
  if (bytes > bytes_) return HipError::copy_failed("host_to_device:size", -1);
  if (bytes == 0) return Unit{};
  const hipError_t e = hipMemcpy(ptr_, src, bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) return HipError::copy_failed("host_to_device", (int32_t)e);
  return Unit{};
}

Result<Unit, HipError> DeviceBuffer::copy_to_host(void* dst, size_t bytes) const {
  if (bytes > bytes_) return HipError::copy_failed("device_to_host:size", -1);
  if (bytes == 0) return Unit{};
  const hipError_t e = hipMemcpy(dst, ptr_, bytes, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return HipError::copy_failed("device_to_host", (int32_t)e);
  return Unit{};
}

size_t DeviceTensor::total_elements() const {
  size_t n = 1;
  for (int64_t d : shape) {
    if (d < 0) return 0;
    if (d != 0 && n > std::numeric_limits<size_t>::max() / (size_t)d)
      return std::numeric_limits<size_t>::max();
    n *= (size_t)d;
  }
  return n;
}

size_t DeviceTensor::byte_size() const {
  const size_t n = total_elements();
  const size_t es = element_size(dtype);
  if (es && n > std::numeric_limits<size_t>::max() / es) return std::numeric_limits<size_t>::max();
  return n * es;
}

bool DeviceTensor::holds_shape() const {
  const size_t n = byte_size();
  if (n == std::numeric_limits<size_t>::max()) return false;
  return buffer.size() >= n && (n == 0 || buffer.as_ptr() != nullptr);
}

Result<DeviceTensor, HipError> DeviceTensor::alloc(std::vector<int64_t> shape, DataType dtype) {
  DeviceTensor t;
  t.shape = std::move(shape);
  t.dtype = dtype;
  auto b = DeviceBuffer::alloc(t.byte_size());
  if (!b) return b.error();
  t.buffer = std::move(b).value();
  return t;
}

Result<DeviceTensor, HipError> DeviceTensor::from_host(const void* raw, size_t bytes,
                                                       std::vector<int64_t> shape,
                                                       DataType dtype, std::string name) {
  auto t = alloc(std::move(shape), dtype);
  if (!t) return t.error();
  if (t.value().byte_size() != bytes) return HipError::copy_failed("host_to_device:size", -1);
  auto c = t.value().buffer.copy_from_host(raw, bytes);
  if (!c) return c.error();
  t.value().name = std::move(name);
  return t;
}

Result<DeviceTensor, HipError> DeviceTensor::from_f32(const std::vector<float>& v,
                                                      std::vector<int64_t> shape) {
  return from_host(v.data(), v.size() * sizeof(float), std::move(shape), DataType::Float);
}

Result<std::vector<uint8_t>, HipError> DeviceTensor::to_host() const {
  std::vector<uint8_t> out(byte_size());
  auto c = buffer.copy_to_host(out.data(), out.size());
  if (!c) return c.error();
  return out;
}

Result<std::vector<float>, HipError> DeviceTensor::to_host_f32() const {
  if (dtype != DataType::Float) return HipError::runtime("to_host_f32:dtype");
  std::vector<float> out(total_elements());
  auto c = buffer.copy_to_host(out.data(), out.size() * sizeof(float));
  if (!c) return c.error();
  return out;
}

// ------------------------------------------------------------------ cache ---
Result<GpuKvCache, HipError> GpuKvCache::allocate(RocmRuntime& rt, size_t num_layers,
                                                  size_t num_kv_heads, size_t head_dim,
                                                  size_t max_seq_len, KvQuant quant,
                                                  const std::vector<LayerKind>& layer_kinds,
                                                  size_t max_batch) {
  if (layer_kinds.size() != num_layers) return HipError::runtime("kv_cache_allocate:layer_kinds_len");
  if (num_layers == 0 || num_kv_heads == 0 || head_dim == 0 || max_seq_len == 0 || max_batch == 0)
    return HipError::runtime("kv_cache_allocate:zero_dim");
  for (const LayerKind& k : layer_kinds)
    if (k.tag == LayerKind::Tag::SlidingWindow &&
        (k.window == 0 || k.window > (size_t)std::numeric_limits<int32_t>::max()))
      return HipError::runtime("kv_cache_allocate:sliding_window");
  const size_t pps = (max_seq_len + SAI_PAGE_TOKENS - 1) / SAI_PAGE_TOKENS;
  const size_t lim = (size_t)std::numeric_limits<int32_t>::max();
  if (num_layers > lim || num_kv_heads > lim || head_dim > lim || pps > lim / max_batch)
    return HipError::alloc_failed(std::numeric_limits<size_t>::max(), -1);
  sai_kvcache_desc d{};
  d.num_layers = (int32_t)num_layers;
  d.num_kv_heads = (int32_t)num_kv_heads;
  d.head_dim = (int32_t)head_dim;
  d.num_pages = (int32_t)(pps * max_batch);
  d.max_batch = (int32_t)max_batch;
  d.max_pages_per_seq = (int32_t)pps;
  d.quant = (int32_t)quant;
  GpuKvCache c;
  c.rt_ = &rt;
  const sai_status st = sai_kvcache_create(rt.raw(), &d, &c.cache_);
  if (st == SAI_ERR_UNSUPPORTED) return HipError::runtime("kv_cache_allocate:unsupported_head_dim", st);
  if (st == SAI_ERR_ALLOC) {
    // block bytes at the stored row width (head_dim 168 is stored 192 wide)
    const size_t sd = head_dim == 168 ? 192 : head_dim;
    const size_t per = quant == KvQuant::Int8 ? 32 * sd + 128 : 20 * sd;
    return HipError::alloc_failed(num_layers * (size_t)d.num_pages * num_kv_heads * per, st);
  }
  if (st != SAI_OK) return HipError::runtime("kv_cache_allocate", st);
  c.num_layers_ = num_layers;
  c.num_kv_heads_ = num_kv_heads;
  c.head_dim_ = head_dim;
  c.max_seq_len_ = max_seq_len;
  c.max_batch_ = max_batch;
  c.pages_per_seq_ = pps;
  c.quant_ = quant;
  c.layer_windows_.assign(num_layers, 0);
  for (size_t l = 0; l < num_layers; ++l) {
    if (layer_kinds[l].tag != LayerKind::Tag::SlidingWindow) continue;
    c.layer_windows_[l] = layer_kinds[l].window;
    const sai_status ws =
        sai_kvcache_set_layer_window(rt.raw(), c.cache_, (int32_t)l, (int32_t)layer_kinds[l].window);
    if (ws != SAI_OK) return HipError::runtime("kv_cache_allocate:sliding_window", ws);
  }
  auto b = c.ensure_batch(max_batch, "kv_cache_allocate");
  if (!b) return b.error();
  return c;
}

GpuKvCache::GpuKvCache(GpuKvCache&& o) noexcept { *this = std::move(o); }

GpuKvCache& GpuKvCache::operator=(GpuKvCache&& o) noexcept {
  if (this != &o) {
    if (cache_) sai_kvcache_destroy(cache_);
    rt_ = o.rt_;
    cache_ = std::exchange(o.cache_, nullptr);
    num_layers_ = o.num_layers_;
    num_kv_heads_ = o.num_kv_heads_;
    head_dim_ = o.head_dim_;
    max_seq_len_ = o.max_seq_len_;
    max_batch_ = o.max_batch_;
    pages_per_seq_ = o.pages_per_seq_;
    layer_windows_ = std::move(o.layer_windows_);
    batch_ = o.batch_;
    position_ = o.position_;
    quant_ = o.quant_;
  }
  return *this;
}

GpuKvCache::~GpuKvCache() {
  if (cache_) {
    // kernels of this cache may still be queued on the device
    (void)hipDeviceSynchronize();
    sai_kvcache_destroy(cache_);
  }
}

size_t GpuKvCache::pending() const {
  int32_t p = 0;
  if (cache_) (void)sai_kvcache_lengths(cache_, nullptr, &p, nullptr);
  return (size_t)p;
}

// Identity page table for `batch` sequences: sequence b owns pages
// [b * pages_per_seq, (b + 1) * pages_per_seq). Only at position 0 with
// nothing pending, since setting a table clears the lengths.
Result<Unit, HipError> GpuKvCache::ensure_batch(size_t batch, const char* op) {
  if (batch == batch_) return Unit{};
  std::string where = std::string(op) + ":batch_mismatch";
  if (batch == 0 || batch > max_batch_ || position_ != 0 || pending() != 0)
    return HipError::runtime(where);
  std::vector<int32_t> pt(batch * pages_per_seq_);
  for (size_t i = 0; i < pt.size(); ++i) pt[i] = (int32_t)i;
  const sai_status st = sai_kvcache_set_page_table(rt_->raw(), cache_, pt.data(), (int32_t)batch);
  if (st != SAI_OK) return HipError::runtime(where, st);
  batch_ = batch;
  return Unit{};
}

Result<Unit, HipError> GpuKvCache::append(size_t layer_idx, const DeviceTensor& new_k,
                                          const DeviceTensor& new_v, const RopeTables* rope,
                                          void* stream) {
  if (layer_idx >= num_layers_) return HipError::runtime("kv_cache_append:layer_idx");
  if (!is_float_like(new_k.dtype) || new_v.dtype != new_k.dtype)
    return HipError::runtime("kv_cache_append:dtype_mismatch");
  const std::vector<int64_t>& s = new_k.shape;
  size_t b = 0, sn = 0;
  if (s.size() == 3 && s[0] > 0 && s[1] > 0 && (size_t)s[2] == num_kv_heads_ * head_dim_) {
    b = (size_t)s[0];
    sn = (size_t)s[1];
  } else if (s.size() == 4 && s[0] > 0 && (size_t)s[1] == num_kv_heads_ && s[2] == 1 &&
             (size_t)s[3] == head_dim_) {
    b = (size_t)s[0];
    sn = 1;
  }
  if (b == 0 || new_v.shape != new_k.shape ||
      new_k.byte_size() != b * sn * num_kv_heads_ * head_dim_ * element_size(new_k.dtype) ||
      !new_k.holds_shape() || !new_v.holds_shape())
    return HipError::runtime("kv_cache_append:tensor_byte_size_mismatch");
  auto ck = check_append(b, sn);
  if (!ck) return ck;
  const sai_status st = sai_kv_append(
      rt_->raw(), cache_, (int32_t)layer_idx, new_k.buffer.as_ptr(), new_v.buffer.as_ptr(),
      sai_dtype(new_k.dtype), (int32_t)b, (int32_t)sn, rope ? rope->cos : nullptr,
      rope ? rope->sin : nullptr, rope ? rope->rows : 0, rope ? 1 : 0,
      rope && rope->interleaved ? 1 : 0, stream);
  if (st != SAI_OK) return HipError::runtime("kv_cache_append: " + rt_->last_error(), st);
  return Unit{};
}

Result<Unit, HipError> GpuKvCache::check_append(size_t batch, size_t s_new) {
  auto eb = ensure_batch(batch, "kv_cache_append");
  if (!eb) return eb;
  if (position_ + s_new > max_seq_len_) return HipError::runtime("kv_cache_append:position_overflow");
  const size_t pend = pending();
  if (pend != 0 && pend != s_new) return HipError::runtime("kv_cache_append:pending_mismatch");
  return Unit{};
}

Result<Unit, HipError> GpuKvCache::advance_position(void* stream) {
  const size_t pend = pending();
  if (pend == 0) return HipError::runtime("kv_cache_advance:nothing_pending");
  if (position_ + pend > max_seq_len_) return HipError::runtime("kv_cache_advance:position_overflow");
  const sai_status st = sai_kvcache_advance(rt_->raw(), cache_, stream);
  if (st != SAI_OK) return HipError::runtime("kv_cache_advance", st);
  position_ += pend;
  return Unit{};
}

Result<KvView, HipError> GpuKvCache::view_at(size_t layer_idx, size_t count, const char* op) const {
  if (layer_idx >= num_layers_) return HipError::runtime(op);
  KvView v;
  void* pool = nullptr;
  const sai_status st =
      sai_kvcache_pool(cache_, (int32_t)layer_idx, &pool, &v.pool_bytes, &v.block_bytes);
  if (st != SAI_OK) return HipError::runtime(op, st);
  v.pool = pool;
  // kv_cache.rs:351-358: a sliding-window layer exposes its last w tokens
  const size_t w = layer_windows_[layer_idx];
  const size_t n = w > 0 ? std::min(w, count) : count;
  v.start_token = count - n;
  v.token_count = n;
  v.num_kv_heads = num_kv_heads_;
  v.head_dim = head_dim_;
  v.batch = batch_;
  v.quant = quant_;
  return v;
}

Result<KvView, HipError> GpuKvCache::view(size_t layer_idx) const {
  return view_at(layer_idx, position_, "kv_cache_view:layer_idx");
}

Result<KvView, HipError> GpuKvCache::view_pending(size_t layer_idx) const {
  return view_at(layer_idx, position_ + pending(), "kv_cache_view_pending:layer_idx");
}

void GpuKvCache::reset() {
  if (cache_) (void)sai_kvcache_reset(rt_->raw(), cache_);
  position_ = 0;
}

Result<std::pair<std::vector<float>, std::vector<float>>, HipError> GpuKvCache::read_dequantized(
    size_t layer_idx, size_t seq, size_t kv_head, size_t t0, size_t n) const {
  if (layer_idx >= num_layers_ || seq >= batch_ || kv_head >= num_kv_heads_)
    return HipError::runtime("kv_cache_read:index");
  if (t0 + n > position_ + pending()) return HipError::runtime("kv_cache_read:range");
  const size_t D = head_dim_;
  std::vector<float> k(n * D), v(n * D);
  if (n == 0) return std::make_pair(std::move(k), std::move(v));
  sai_status st;
  if (quant_ == KvQuant::Int8) {
    std::vector<int8_t> kc(n * D), vc(n * D);
    std::vector<float> ks(n), vs(n);
    st = sai_kvcache_read(rt_->raw(), cache_, (int32_t)layer_idx, (int32_t)seq, (int32_t)kv_head,
                          (int32_t)t0, (int32_t)n, kc.data(), vc.data(), ks.data(), vs.data());
    if (st != SAI_OK) return HipError::runtime("kv_cache_read", st);
    for (size_t t = 0; t < n; ++t)
      for (size_t d = 0; d < D; ++d) {
        k[t * D + d] = (float)kc[t * D + d] * ks[t];
        v[t * D + d] = (float)vc[t * D + d] * vs[t];
      }
  } else {
    const size_t G = D / 32;
    std::vector<uint8_t> kc(n * D / 2), vc(n * D / 2);
    std::vector<uint16_t> kp(n * G * 2), vp(n * G * 2);
    st = sai_kvcache_read(rt_->raw(), cache_, (int32_t)layer_idx, (int32_t)seq, (int32_t)kv_head,
                          (int32_t)t0, (int32_t)n, kc.data(), vc.data(), kp.data(), vp.data());
    if (st != SAI_OK) return HipError::runtime("kv_cache_read", st);
    for (size_t t = 0; t < n; ++t)
      for (size_t d = 0; d < D; ++d) {
        const size_t g = d / 32;
        const uint8_t kb = kc[t * D / 2 + d / 2], vb = vc[t * D / 2 + d / 2];
        const float kq = (float)((d & 1) ? kb >> 4 : kb & 0xF);
        const float vq = (float)((d & 1) ? vb >> 4 : vb & 0xF);
        // code * scale + zero, each rounded on its own
        const float ka = kq * half_to_float(kp[(t * G + g) * 2]);
        const float va = vq * half_to_float(vp[(t * G + g) * 2]);
        k[t * D + d] = ka + half_to_float(kp[(t * G + g) * 2 + 1]);
        v[t * D + d] = va + half_to_float(vp[(t * G + g) * 2 + 1]);
      }
  }
  return std::make_pair(std::move(k), std::move(v));
}

// ------------------------------------------------------------- operator ---
AttributeProto AttributeProto::make_int(std::string n, int64_t v) {
  AttributeProto a;
  a.name = std::move(n);
  a.attr_type = AttributeType::Int;
  a.i = v;
  return a;
}

AttributeProto AttributeProto::make_float(std::string n, float v) {
  AttributeProto a;
  a.name = std::move(n);
  a.attr_type = AttributeType::Float;
  a.f = v;
  return a;
}

GqaAttrs parse_gqa_attrs(const std::vector<AttributeProto>& attrs) {
  GqaAttrs a;
  // first attribute of a name and type wins (executor.rs:350-365)
  bool seen_nh = false, seen_kv = false, seen_lw = false, seen_rot = false, seen_il = false;
  for (const AttributeProto& p : attrs) {
    if (p.attr_type == AttributeType::Int) {
      if (p.name == "num_heads" && !seen_nh) {
        a.num_heads = p.i;
        seen_nh = true;
      } else if (p.name == "kv_num_heads" && !seen_kv) {
        a.kv_num_heads = p.i;
        seen_kv = true;
      } else if (p.name == "local_window_size" && !seen_lw) {
        a.local_window_size = p.i;
        seen_lw = true;
      } else if (p.name == "do_rotary" && !seen_rot) {
        a.do_rotary = p.i != 0;
        a.do_rotary_set = true;
        seen_rot = true;
      } else if (p.name == "rotary_interleaved" && !seen_il) {
        a.rotary_interleaved = p.i != 0;
        seen_il = true;
      }
    } else if (p.attr_type == AttributeType::Float && p.name == "scale" && !a.scale) {
      a.scale = p.f;
    }
  }
  return a;
}

Result<GqaShape, OpError> gqa_validate(const std::vector<int64_t>& q, const std::vector<int64_t>& k,
                                       const std::vector<int64_t>& v, int64_t num_heads,
                                       int64_t kv_num_heads) {
  GqaShape g;
  if (q.size() == 4 && k.size() == 4 && v.size() == 4) {
    // [B, H, S, D]: heads from the shapes (gpu_gqa's rank-4 contract)
    if (q[1] <= 0 || k[1] <= 0)
      return OpError::attribute("GroupQueryAttention: num_heads and kv_num_heads must be > 0");
    if (q[1] % k[1] != 0)
      return OpError::attribute("GroupQueryAttention: num_heads must be a multiple of kv_num_heads");
    if (q[0] < 0 || q[2] < 0 || q[3] <= 0)
      return OpError::shape("GroupQueryAttention: Q/K/V must be rank-3");
    if (k[3] != q[3]) return OpError::shape("GroupQueryAttention: Q and KV head_dim must match");
    if (v != k) return OpError::shape("GroupQueryAttention: key and value must have the same shape");
    if (q[2] != 1 || k[2] != 1 || k[0] != q[0])
      return OpError::shape("GroupQueryAttention: rank-4 [B, H, S, D] inputs need S = 1 (decode)");
    g.num_heads = (size_t)q[1];
    g.kv_heads = (size_t)k[1];
    g.batch = (size_t)q[0];
    g.seq = 1;
    g.head_dim = (size_t)q[3];
    g.q_hidden = g.num_heads * g.head_dim;
    return g;
  }
  if (num_heads <= 0 || kv_num_heads <= 0)
    return OpError::attribute("GroupQueryAttention: num_heads and kv_num_heads must be > 0");
  if (num_heads % kv_num_heads != 0)
    return OpError::attribute("GroupQueryAttention: num_heads must be a multiple of kv_num_heads");
  if (q.size() != 3 || k.size() != 3 || v.size() != 3)
    return OpError::shape("GroupQueryAttention: Q/K/V must be rank-3");
  if (q[0] < 0 || q[1] < 0 || q[2] < 0 || k[2] < 0)
    return OpError::shape("GroupQueryAttention: Q/K/V must be rank-3");
  const size_t nh = (size_t)num_heads, kvh = (size_t)kv_num_heads;
  const size_t q_hidden = (size_t)q[2], kv_hidden = (size_t)k[2];
  if (q_hidden % nh != 0)
    return OpError::shape("GroupQueryAttention: q_hidden not divisible by num_heads");
  if (kv_hidden % kvh != 0)
    return OpError::shape("GroupQueryAttention: kv_hidden not divisible by kv_num_heads");
  const size_t head_dim = q_hidden / nh;
  if (kv_hidden / kvh != head_dim)
    return OpError::shape("GroupQueryAttention: Q and KV head_dim must match");
  if (v != k) return OpError::shape("GroupQueryAttention: key and value must have the same shape");
  // the op reads K/V with Q's batch and sequence (reshape_to_bhsd(key, b, sq, ...))
  if (k[0] != q[0] || k[1] != q[1])
    return OpError::shape("GroupQueryAttention: key batch/sequence must match query");
  g.num_heads = nh;
  g.kv_heads = kvh;
  g.batch = (size_t)q[0];
  g.seq = (size_t)q[1];
  g.q_hidden = q_hidden;
  g.head_dim = head_dim;
  return g;
}

namespace {

const DeviceTensor* slot(const std::vector<const DeviceTensor*>& in, size_t i) {
  return i < in.size() ? in[i] : nullptr;
}

// validate_rope_caches (ops/microsoft.rs:71-110) with rotary_dim = head_dim.
Result<int32_t, OpError> check_rope_tables(const DeviceTensor& cos, const DeviceTensor& sin,
                                           size_t head_dim) {
  if (cos.dtype != DataType::Float || sin.dtype != DataType::Float)
    return OpError::shape("RotaryEmbedding requires Float input");
  if (head_dim % 2 != 0)
    return OpError::attribute("apply_rope_in_place: rotary_dim must be even");
  if (cos.shape.size() != 2 || sin.shape.size() != 2)
    return OpError::shape("apply_rope_in_place: cos/sin caches must be rank-2");
  if (sin.shape[1] != cos.shape[1])
    return OpError::shape("apply_rope_in_place: cos and sin caches must share the inner dim");
  if (cos.shape[1] != (int64_t)(head_dim / 2)) {
    char buf[128];
    std::snprintf(buf, sizeof buf, "apply_rope_in_place: cache inner dim %lld != rotary_dim/2 = %zu",
                  (long long)cos.shape[1], head_dim / 2);
    return OpError::shape(buf);
  }
  // both tables are read at the same rows
  const int64_t rows = std::min(cos.shape[0], sin.shape[0]);
  if (rows < 0 || rows > std::numeric_limits<int32_t>::max())
    return OpError::shape("apply_rope_in_place: cos/sin caches must be rank-2");
  if (!cos.holds_shape() || !sin.holds_shape())
    return OpError::shape("apply_rope_in_place: cos/sin buffer does not hold its shape");
  return (int32_t)rows;
}

OpError from_status(sai_status st, const std::string& prefix, const RocmRuntime& rt) {
  return OpError{kind_of(st), prefix + rt.last_error()};
}

// One GQA node over `cache` (layer `layer`): fused append + decode for S = 1,
// append + prefill chunk for S > 1.
Result<DeviceTensor, OpError> gqa_over_cache(RocmRuntime& rt, GpuKvCache& cache, size_t layer,
                                             const DeviceTensor& q, const DeviceTensor& k,
                                             const DeviceTensor& v, const GqaShape& g,
                                             const GqaAttrs& a, const RopeTables* rope,
                                             const std::string& prefix) {
  if (g.kv_heads != cache.num_kv_heads() || g.head_dim != cache.head_dim())
    return OpError::shape(prefix + "K/V heads or head_dim differ from the cache's");
  // attn_out takes Q's dtype, as the reference's GPU attention does
  // (gpu_gqa's dt = q.dtype and its bf16 PV GEMM + gqa_merge_heads_bf16,
  // cuda/kernels/attention.rs:835, :877-901, :495-520)
  auto out = DeviceTensor::alloc({(int64_t)g.batch, (int64_t)g.seq, (int64_t)g.q_hidden},
                                 q.dtype);
  if (!out) return OpError::internal(prefix + out.error().to_string());
  if (g.batch == 0 || g.seq == 0) return std::move(out).value();
  const float* cs = rope ? rope->cos : nullptr;
  const float* sn = rope ? rope->sin : nullptr;
  const int32_t rows = rope ? rope->rows : 0;
  const int32_t rot = rope ? 1 : 0;
  const int32_t il = a.rotary_interleaved ? 1 : 0;
  const int32_t has_scale = a.scale ? 1 : 0;
  const float scale = a.scale ? *a.scale : 0.0f;
  // parse_gqa_attrs (gpu_executor.rs:874-878): a positive local_window_size
  // is the kernel's window, anything else none
  const int32_t window = a.local_window_size > 0
                             ? (int32_t)std::min<int64_t>(a.local_window_size,
                                                          std::numeric_limits<int32_t>::max())
                             : 0;
  void* o = out.value().buffer.as_ptr();
  const int32_t odt = sai_dtype(q.dtype);
  if (g.seq == 1) {
    auto ck = cache.check_append(g.batch, 1);
    if (!ck) return OpError::internal(prefix + ck.error().to_string());
    const sai_status st = sai_gqa_with_cache(
        rt.raw(), cache.raw(), (int32_t)layer, q.buffer.as_ptr(), sai_dtype(q.dtype),
        k.buffer.as_ptr(), v.buffer.as_ptr(), sai_dtype(k.dtype), (int32_t)g.batch,
        (int32_t)g.num_heads, cs, sn, rows, rot, il, has_scale, scale, window, o, odt, nullptr);
    if (st != SAI_OK) return from_status(st, prefix, rt);
    return std::move(out).value();
  }
  auto ap = cache.append(layer, k, v, rope, nullptr);
  if (!ap) return OpError::internal(prefix + ap.error().to_string());
  const sai_status st = sai_gqa_prefill(rt.raw(), cache.raw(), (int32_t)layer, q.buffer.as_ptr(),
                                        sai_dtype(q.dtype), (int32_t)g.batch, (int32_t)g.seq,
                                        (int32_t)g.num_heads, cs, sn, rows, rot, il, has_scale,
                                        scale, window, o, odt, nullptr);
  if (st != SAI_OK) return from_status(st, prefix, rt);
  return std::move(out).value();
}

}  // namespace

Result<std::vector<DeviceTensor>, OpError> dispatch_gqa(
    RocmRuntime& runtime, const std::vector<const DeviceTensor*>& inputs,
    const std::vector<AttributeProto>& attrs, KvCacheDispatchCtx* kv_cache_ctx) {
  static const char* const roles[3] = {"Q", "K", "V"};
  for (size_t i = 0; i < 3; ++i)
    if (!slot(inputs, i))
      return OpError::internal(std::string("GPU GroupQueryAttention: missing input '") + roles[i] + "'");
  const DeviceTensor& q = *inputs[0];
  const DeviceTensor& k = *inputs[1];
  const DeviceTensor& v = *inputs[2];
  const GqaAttrs a = parse_gqa_attrs(attrs);
  auto gs = gqa_validate(q.shape, k.shape, v.shape, a.num_heads, a.kv_num_heads);
  if (!gs) return gs.error();
  const GqaShape g = gs.value();
  if (!is_float_like(q.dtype) || !is_float_like(k.dtype) || v.dtype != k.dtype)
    return OpError::shape("GroupQueryAttention requires Float or BFloat16 input");
  if (q.byte_size() != g.batch * g.seq * g.q_hidden * element_size(q.dtype) ||
      k.byte_size() != g.batch * g.seq * g.kv_heads * g.head_dim * element_size(k.dtype) ||
      !q.holds_shape() || !k.holds_shape() || !v.holds_shape())
    return OpError::shape("GroupQueryAttention: input buffer does not hold its shape");

  // RoPE tables (inputs 7 and 8, gqa_apply_rotary, ops/microsoft.rs:1004-1020)
  const DeviceTensor* cos = slot(inputs, 7);
  const DeviceTensor* sin = slot(inputs, 8);
  RopeTables rope;
  const RopeTables* rope_ptr = nullptr;
  if (a.do_rotary && (a.do_rotary_set || cos || sin)) {
    if (!cos) return OpError::shape("GroupQueryAttention: do_rotary=1 but cos_cache is missing");
    if (!sin) return OpError::shape("GroupQueryAttention: do_rotary=1 but sin_cache is missing");
    auto rows = check_rope_tables(*cos, *sin, g.head_dim);
    if (!rows) return rows.error();
    rope.cos = (const float*)cos->buffer.as_ptr();
    rope.sin = (const float*)sin->buffer.as_ptr();
    rope.rows = rows.value();
    rope.interleaved = a.rotary_interleaved;
    rope_ptr = &rope;
  }

  if (kv_cache_ctx && kv_cache_ctx->cache) {
    const size_t layer = kv_cache_ctx->next_layer_idx++;
    auto r = gqa_over_cache(runtime, *kv_cache_ctx->cache, layer, q, k, v, g, a, rope_ptr,
                            "ROCm GroupQueryAttention (cache): ");
    if (!r) return r.error();
    std::vector<DeviceTensor> outs;
    outs.push_back(std::move(r).value());
    return outs;
  }

  // No cache: attention over the node's own K/V (gqa_cacheless,
  // gpu_executor.rs:933-942), through a transient one-layer cache.
  const std::string prefix = "ROCm GroupQueryAttention: ";
  if (g.batch == 0 || g.seq == 0) {
    auto out = DeviceTensor::alloc({(int64_t)g.batch, (int64_t)g.seq, (int64_t)g.q_hidden},
                                   q.dtype);
    if (!out) return OpError::internal(prefix + out.error().to_string());
    std::vector<DeviceTensor> outs;
    outs.push_back(std::move(out).value());
    return outs;
  }
  auto cache = GpuKvCache::allocate(runtime, 1, g.kv_heads, g.head_dim, g.seq, KvQuant::Int8,
                                    {LayerKind::global()}, g.batch);
  if (!cache) {
    const HipError& e = cache.error();
    if (e.op == "kv_cache_allocate:unsupported_head_dim")
      return OpError::unsupported(prefix + e.to_string());
    return OpError::internal(prefix + e.to_string());
  }
  auto r = gqa_over_cache(runtime, cache.value(), 0, q, k, v, g, a, rope_ptr, prefix);
  if (!r) return r.error();
  // the transient cache is freed on return, after the device has drained
  std::vector<DeviceTensor> outs;
  outs.push_back(std::move(r).value());
  return outs;
}

// --------------------------------------------------------- RotaryEmbedding ---
namespace {

// find_int_attr (gpu_executor.rs:701-703): the first attribute of that name.
const AttributeProto* find_attr(const std::vector<AttributeProto>& attrs, const char* name) {
  for (const AttributeProto& a : attrs)
    if (a.name == name) return &a;
  return nullptr;
}

bool is_table_dtype(DataType dt) { return dt == DataType::Float || dt == DataType::BFloat16; }

OpError rotary_gpu_error(const char* what) {
  return OpError::internal(std::string("ROCm RotaryEmbedding: ") +
                           HipError::runtime(what).to_string());
}

// The host copy of a device tensor's bytes.
Result<std::vector<uint8_t>, OpError> read_back(const DeviceTensor& t, const char* what) {
  auto h = t.to_host();
  if (!h) return OpError::internal(std::string(what) + ": " + h.error().to_string());
  return std::move(h).value();
}

}  // namespace

Result<std::vector<DeviceTensor>, OpError> dispatch_rotary_embedding(
    RocmRuntime& runtime, const std::vector<const DeviceTensor*>& inputs,
    const std::vector<AttributeProto>& attrs, const KvCacheDispatchCtx* kv_cache_ctx) {
  auto missing = [](const char* role) {
    return OpError::internal(std::string("GPU RotaryEmbedding: missing input '") + role + "'");
  };
  const DeviceTensor* x = slot(inputs, 0);
  if (!x) return missing("X");
  // resolve_rotary_inputs (gpu_executor.rs:724-745)
  const DeviceTensor *pos = nullptr, *cos = nullptr, *sin = nullptr;
  if (inputs.size() >= 4) {
    if (!(pos = slot(inputs, 1))) return missing("position_ids");
    if (!(cos = slot(inputs, 2))) return missing("cos_cache");
    if (!(sin = slot(inputs, 3))) return missing("sin_cache");
  } else {
    if (!(cos = slot(inputs, 1))) return missing("cos_cache");
    if (!(sin = slot(inputs, 2))) return missing("sin_cache");
  }
  if (!x->holds_shape() || !cos->holds_shape() || !sin->holds_shape() ||
      (pos && !pos->holds_shape()))
    return OpError::shape("GPU RotaryEmbedding: input buffer does not hold its shape");
  const AttributeProto* il = find_attr(attrs, "interleaved");
  const bool interleaved = il && il->i != 0;
  // pick_rotary_position / read_first_i64_position (gpu_executor.rs:747-771)
  int32_t position = 0;
  if (pos) {
    auto raw = read_back(*pos, "RotaryEmbedding pos D2H");
    if (!raw) return raw.error();
    const std::vector<uint8_t>& b = raw.value();
    if (b.size() >= 8) {
      int64_t v;
      std::memcpy(&v, b.data(), 8);
      position = (int32_t)(uint32_t)(uint64_t)v;  // `as i32`: the low 32 bits
    }
  } else if (kv_cache_ctx && kv_cache_ctx->cache) {
    position = (int32_t)kv_cache_ctx->cache->current_position();
  }
  // rotary_num_heads_for_rank3 (gpu_executor.rs:795-813)
  std::optional<int64_t> nh3;
  if (x->shape.size() == 3) {
    if (const AttributeProto* nh = find_attr(attrs, "num_heads")) {
      nh3 = nh->i;
    } else {
      const int64_t hd = (cos->shape.empty() ? 0 : cos->shape.back()) * 2;
      if (hd > 0 && x->shape[2] % hd == 0) nh3 = x->shape[2] / hd;
    }
  }
  // rotary_gpu (kernels/rotary.rs:274-374)
  if (x->dtype != DataType::Float && x->dtype != DataType::BFloat16)
    return rotary_gpu_error("rotary_gpu: unsupported dtype (need Float or BFloat16)");
  int64_t B, H, S, D;
  int32_t layout;
  if (x->shape.size() == 4) {
    B = x->shape[0], H = x->shape[1], S = x->shape[2], D = x->shape[3];
    layout = SAI_ROPE_BHSD;
  } else if (x->shape.size() == 3) {
    if (!nh3) return rotary_gpu_error("rotary_gpu: rank-3 input requires num_heads_for_rank3");
    if (*nh3 <= 0) return rotary_gpu_error("rotary_gpu: num_heads must be > 0 for rank-3 input");
    if (x->shape[2] % *nh3 != 0)
      return rotary_gpu_error("rotary_gpu: hidden not divisible by num_heads (rank-3)");
    B = x->shape[0], H = *nh3, S = x->shape[1], D = x->shape[2] / *nh3;
    layout = SAI_ROPE_BSHD;
  } else {
    return rotary_gpu_error("rotary_gpu: x must be rank-3 or rank-4");
  }
  if (D <= 0 || D % 2 != 0)
    return rotary_gpu_error("rotary_gpu: head_dim must be a positive even integer");
  const int64_t half = D / 2;
  // validate_rotary_tables (rotary.rs:218-256); bf16 tables count as Float,
  // as the reference casts them first
  if (!is_table_dtype(cos->dtype) || !is_table_dtype(sin->dtype))
    return rotary_gpu_error("rotary_gpu: cos/sin tables must be Float");
  if (cos->shape.size() != 2 || sin->shape.size() != 2)
    return rotary_gpu_error("rotary_gpu: cos/sin tables must be rank-2");
  if (cos->shape[1] != half || sin->shape[1] != half)
    return rotary_gpu_error("rotary_gpu: cos/sin inner dim must equal head_dim / 2");
  const int64_t max_seq = cos->shape[0];
  if (sin->shape[0] != max_seq)
    return rotary_gpu_error("rotary_gpu: cos/sin tables must share max_seq_len");
  if (position < 0 || (int64_t)position + S > max_seq)
    return rotary_gpu_error("rotary_gpu: position + seq_len exceeds cos/sin table length");
  if (cos->dtype != sin->dtype)
    return rotary_gpu_error("rotary_gpu: cos/sin tables must share a dtype");
  auto out = DeviceTensor::alloc(x->shape, x->dtype);
  if (!out) return OpError::internal("ROCm RotaryEmbedding: " + out.error().to_string());
  std::vector<DeviceTensor> outs;
  if (B <= 0 || H <= 0 || S <= 0) {
    outs.push_back(std::move(out).value());
    return outs;
  }
  const int64_t lim = std::numeric_limits<int32_t>::max();
  if (B > lim || H > lim || S > lim || D > lim || max_seq > lim)
    return rotary_gpu_error("rotary_gpu: dimension exceeds i32");
  const sai_status st = sai_rotary_embedding(
      runtime.raw(), x->buffer.as_ptr(), out.value().buffer.as_ptr(), sai_dtype(x->dtype),
      (int32_t)B, (int32_t)H, (int32_t)S, (int32_t)D, layout, nullptr, 0, position,
      cos->buffer.as_ptr(), sin->buffer.as_ptr(), sai_dtype(cos->dtype), (int32_t)max_seq,
      (int32_t)half, (int32_t)D, interleaved ? 1 : 0, nullptr);
  if (st != SAI_OK) return from_status(st, "ROCm RotaryEmbedding: ", runtime);
  outs.push_back(std::move(out).value());
  return outs;
}

Result<DeviceTensor, OpError> op_rotary_embedding(RocmRuntime& runtime,
                                                  const std::vector<const DeviceTensor*>& inputs,
                                                  bool interleaved, int64_t rotary_embedding_dim,
                                                  int64_t num_heads_attr) {
  const DeviceTensor* input = slot(inputs, 0);
  if (!input) return OpError::shape("RotaryEmbedding: missing input");
  const DeviceTensor* position_ids = slot(inputs, 1);
  if (!position_ids) return OpError::shape("RotaryEmbedding: missing position_ids");
  const DeviceTensor* cos = slot(inputs, 2);
  if (!cos) return OpError::shape("RotaryEmbedding: missing cos_cache");
  const DeviceTensor* sin = slot(inputs, 3);
  if (!sin) return OpError::shape("RotaryEmbedding: missing sin_cache");
  if (!input->holds_shape() || !position_ids->holds_shape() || !cos->holds_shape() ||
      !sin->holds_shape())
    return OpError::shape("RotaryEmbedding: input buffer does not hold its shape");
  if (input->dtype != DataType::Float) return OpError::shape("RotaryEmbedding requires Float input");
  // rank 3 is read as [B, num_heads, S, D] over the same bytes (microsoft.rs:578-600)
  std::vector<int64_t> view;
  if (input->shape.size() == 3) {
    const int64_t b = input->shape[0], sq = input->shape[1], hidden = input->shape[2];
    if (num_heads_attr <= 0)
      return OpError::attribute("RotaryEmbedding: num_heads must be > 0 for rank-3 input");
    if (hidden % num_heads_attr != 0)
      return OpError::shape("RotaryEmbedding: hidden not divisible by num_heads");
    view = {b, num_heads_attr, sq, hidden / num_heads_attr};
  } else if (input->shape.size() == 4) {
    view = input->shape;
  } else {
    return OpError::shape("RotaryEmbedding: input must be rank-3 or rank-4");
  }
  for (int64_t v : view)
    if (v < 0 || v > std::numeric_limits<int32_t>::max())
      return OpError::shape("RotaryEmbedding: dimension out of range");
  const int64_t head_dim = view[3];
  const int64_t rotary_dim = rotary_embedding_dim <= 0 ? head_dim : rotary_embedding_dim;
  std::vector<int64_t> positions;
  if (position_ids->dtype == DataType::Int64 || position_ids->dtype == DataType::Int32) {
    auto raw = read_back(*position_ids, "RotaryEmbedding position_ids D2H");
    if (!raw) return raw.error();
    const std::vector<uint8_t>& b = raw.value();
    const size_t n = position_ids->total_elements();
    positions.resize(n);
    for (size_t i = 0; i < n; ++i) {
      if (position_ids->dtype == DataType::Int64) {
        std::memcpy(&positions[i], b.data() + 8 * i, 8);
      } else {
        int32_t v;
        std::memcpy(&v, b.data() + 4 * i, 4);
        positions[i] = v;
      }
    }
  } else {
    return OpError::shape("RotaryEmbedding: position_ids must be int32 or int64");
  }
  // apply_rope_in_place (microsoft.rs:177-233) with validate_rope_caches (:71-110)
  const int64_t b = view[0], sq = view[2];
  if ((int64_t)positions.size() != b * sq && (int64_t)positions.size() != sq) {
    char buf[160];
    std::snprintf(buf, sizeof buf, "apply_rope_in_place: position_ids length %zu != B*Sq = %lld",
                  positions.size(), (long long)(b * sq));
    return OpError::shape(buf);
  }
  if (cos->dtype != DataType::Float || sin->dtype != DataType::Float)
    return OpError::shape("RotaryEmbedding requires Float input");
  if (rotary_dim == 0 || rotary_dim > head_dim)
    return OpError::attribute("apply_rope_in_place: rotary_dim must be in 1..=head_dim");
  if (rotary_dim % 2 != 0) return OpError::attribute("apply_rope_in_place: rotary_dim must be even");
  if (cos->shape.size() != 2 || sin->shape.size() != 2)
    return OpError::shape("apply_rope_in_place: cos/sin caches must be rank-2");
  if (sin->shape[1] != cos->shape[1])
    return OpError::shape("apply_rope_in_place: cos and sin caches must share the inner dim");
  if (cos->shape[1] != rotary_dim / 2) {
    char buf[128];
    std::snprintf(buf, sizeof buf, "apply_rope_in_place: cache inner dim %lld != rotary_dim/2 = %lld",
                  (long long)cos->shape[1], (long long)(rotary_dim / 2));
    return OpError::shape(buf);
  }
  // both tables are read at the same rows
  const int64_t rows = std::min(cos->shape[0], sin->shape[0]);
  if (rows < 0 || rows > std::numeric_limits<int32_t>::max())
    return OpError::shape("apply_rope_in_place: cos/sin caches must be rank-2");
  auto out = DeviceTensor::alloc(input->shape, DataType::Float);
  if (!out) return OpError::internal("ROCm RotaryEmbedding: " + out.error().to_string());
  const sai_status st = sai_rotary_embedding(
      runtime.raw(), input->buffer.as_ptr(), out.value().buffer.as_ptr(), SAI_DTYPE_F32,
      (int32_t)view[0], (int32_t)view[1], (int32_t)view[2], (int32_t)view[3], SAI_ROPE_BHSD,
      positions.data(), (int64_t)positions.size(), 0, cos->buffer.as_ptr(), sin->buffer.as_ptr(),
      SAI_DTYPE_F32, (int32_t)rows, (int32_t)cos->shape[1], (int32_t)rotary_dim,
      interleaved ? 1 : 0, nullptr);
  if (st != SAI_OK) return from_status(st, "", runtime);
  return std::move(out).value();
}

Result<std::pair<DeviceTensor, DeviceTensor>, HipError> precompute_rope_tables(
    RocmRuntime& runtime, size_t max_pos, size_t half, float rope_theta) {
  if (max_pos > (size_t)std::numeric_limits<int32_t>::max() ||
      half > (size_t)std::numeric_limits<int32_t>::max())
    return HipError::runtime("precompute_rope_tables:size", SAI_ERR_UNSUPPORTED);
  auto c = DeviceTensor::alloc({(int64_t)max_pos, (int64_t)half}, DataType::BFloat16);
  if (!c) return c.error();
  auto s = DeviceTensor::alloc({(int64_t)max_pos, (int64_t)half}, DataType::BFloat16);
  if (!s) return s.error();
  const sai_status st =
      sai_rope_tables(runtime.raw(), rope_theta, (int32_t)max_pos, (int32_t)half, SAI_DTYPE_BF16,
                      c.value().buffer.as_ptr(), s.value().buffer.as_ptr(), nullptr);
  if (st != SAI_OK) return HipError::runtime("precompute_rope_tables", st);
  return std::make_pair(std::move(c).value(), std::move(s).value());
}

// ------------------------------------------------- CPU attention op contracts ---
namespace {

OpError shape_fmt(const char* fmt, long long a, long long b) {
  char buf[192];
  std::snprintf(buf, sizeof buf, fmt, a, b);
  return OpError::shape(buf);
}

// validate_past_kv (ops/microsoft.rs:707-731): the past's sequence length.
Result<size_t, OpError> validate_past_kv(const DeviceTensor* past, size_t batch, size_t heads,
                                         size_t head_dim) {
  if (!past) return (size_t)0;
  if (past->dtype != DataType::Float) return OpError::shape("GroupQueryAttention requires Float input");
  if (past->shape.size() != 4)
    return OpError::shape("GQA/MHA: past_key/past_value must be rank-4");
  if (past->shape[0] != (int64_t)batch || past->shape[1] != (int64_t)heads ||
      past->shape[3] != (int64_t)head_dim || past->shape[2] < 0)
    return OpError::shape("GQA/MHA: past cache batch/heads/head_dim mismatch");
  if (!past->holds_shape())
    return OpError::shape("GQA/MHA: past cache buffer does not hold its shape");
  return (size_t)past->shape[2];
}

Result<DeviceTensor, OpError> alloc_or(std::vector<int64_t> shape, DataType dt,
                                       const std::string& prefix) {
  auto t = DeviceTensor::alloc(std::move(shape), dt);
  if (!t) return OpError::internal(prefix + t.error().to_string());
  return std::move(t).value();
}

// Shared GPU path of the two ops. q [B, S, Hq*D], k/v [B, S, Hkv*D] (f32),
// past_k/past_v [B, Hkv, P, D] or null (P == 0).
Result<AttentionOutputs, OpError> attention_with_past(
    RocmRuntime& rt, const DeviceTensor& q, const DeviceTensor& k, const DeviceTensor& v,
    const DeviceTensor* past_k, const DeviceTensor* past_v, size_t P, const GqaShape& g,
    const RopeTables* rope, std::optional<float> scale, const std::string& prefix) {
  const size_t B = g.batch, S = g.seq, Hkv = g.kv_heads, D = g.head_dim, T = P + S;
  const int64_t lim = std::numeric_limits<int32_t>::max();
  if ((int64_t)T > lim || (int64_t)(B * Hkv) > lim)
    return OpError::unsupported(prefix + "sequence or batch too large");
  auto pk = alloc_or({(int64_t)B, (int64_t)Hkv, (int64_t)T, (int64_t)D}, DataType::Float, prefix);
  if (!pk) return pk.error();
  auto pv = alloc_or({(int64_t)B, (int64_t)Hkv, (int64_t)T, (int64_t)D}, DataType::Float, prefix);
  if (!pv) return pv.error();
  auto attn = alloc_or({(int64_t)B, (int64_t)S, (int64_t)g.q_hidden}, DataType::Float, prefix);
  if (!attn) return attn.error();
  sai_ctx* ctx = rt.raw();
  auto copy = [&](const void* src, int32_t src_layout, void* dst, int32_t seq, int32_t off) {
    return sai_copy_rows(ctx, src, src_layout, dst, SAI_ROPE_BHSD, SAI_DTYPE_F32, (int32_t)B,
                         (int32_t)Hkv, seq, (int32_t)D, (int32_t)T, off, nullptr);
  };
  // present = past ++ new (kv_concat, microsoft.rs:762-792), new K rotated first
  sai_status st = SAI_OK;
  if (P > 0) {
    st = copy(past_k->buffer.as_ptr(), SAI_ROPE_BHSD, pk.value().buffer.as_ptr(), (int32_t)P, 0);
    if (st == SAI_OK)
      st = copy(past_v->buffer.as_ptr(), SAI_ROPE_BHSD, pv.value().buffer.as_ptr(), (int32_t)P, 0);
    if (st != SAI_OK) return from_status(st, prefix, rt);
  }
  DeviceTensor k_rot;
  const void* k_new = k.buffer.as_ptr();
  if (rope && B * S > 0) {
    auto kr = alloc_or(k.shape, DataType::Float, prefix);
    if (!kr) return kr.error();
    k_rot = std::move(kr).value();
    st = sai_rotary_embedding(ctx, k.buffer.as_ptr(), k_rot.buffer.as_ptr(), SAI_DTYPE_F32,
                              (int32_t)B, (int32_t)Hkv, (int32_t)S, (int32_t)D, SAI_ROPE_BSHD,
                              nullptr, 0, (int64_t)P, rope->cos, rope->sin, SAI_DTYPE_F32,
                              rope->rows, (int32_t)(D / 2), (int32_t)D, rope->interleaved ? 1 : 0,
                              nullptr);
    if (st != SAI_OK) return from_status(st, prefix, rt);
    k_new = k_rot.buffer.as_ptr();
  }
  st = copy(k_new, SAI_ROPE_BSHD, pk.value().buffer.as_ptr(), (int32_t)S, (int32_t)P);
  if (st == SAI_OK) st = copy(v.buffer.as_ptr(), SAI_ROPE_BSHD, pv.value().buffer.as_ptr(), (int32_t)S, (int32_t)P);
  if (st != SAI_OK) return from_status(st, prefix, rt);
  AttentionOutputs out{std::move(attn).value(), std::move(pk).value(), std::move(pv).value()};
  if (B == 0 || S == 0) return out;

  // attention over a transient paged cache: the past (already rotated) first,
  // committed; then the new tokens through the fused decode or append + prefill
  auto cache = GpuKvCache::allocate(rt, 1, Hkv, D, T, KvQuant::Int8, {LayerKind::global()}, B);
  if (!cache) {
    const HipError& e = cache.error();
    if (e.op == "kv_cache_allocate:unsupported_head_dim")
      return OpError::unsupported(prefix + e.to_string());
    return OpError::internal(prefix + e.to_string());
  }
  if (P > 0) {
    auto rk = alloc_or({(int64_t)B, (int64_t)P, (int64_t)(Hkv * D)}, DataType::Float, prefix);
    if (!rk) return rk.error();
    auto rv = alloc_or({(int64_t)B, (int64_t)P, (int64_t)(Hkv * D)}, DataType::Float, prefix);
    if (!rv) return rv.error();
    auto to_rows = [&](const void* src, void* dst) {
      return sai_copy_rows(ctx, src, SAI_ROPE_BHSD, dst, SAI_ROPE_BSHD, SAI_DTYPE_F32, (int32_t)B,
                           (int32_t)Hkv, (int32_t)P, (int32_t)D, (int32_t)P, 0, nullptr);
    };
    st = to_rows(past_k->buffer.as_ptr(), rk.value().buffer.as_ptr());
    if (st == SAI_OK) st = to_rows(past_v->buffer.as_ptr(), rv.value().buffer.as_ptr());
    if (st != SAI_OK) return from_status(st, prefix, rt);
    auto ap = cache.value().append(0, rk.value(), rv.value(), nullptr, nullptr);
    if (!ap) return OpError::internal(prefix + ap.error().to_string());
    auto adv = cache.value().advance_position(nullptr);
    if (!adv) return OpError::internal(prefix + adv.error().to_string());
  }
  GqaAttrs a;
  a.num_heads = (int64_t)g.num_heads;
  a.kv_num_heads = (int64_t)Hkv;
  a.scale = scale;
  a.rotary_interleaved = rope && rope->interleaved;
  auto r = gqa_over_cache(rt, cache.value(), 0, q, k, v, g, a, rope, prefix);
  if (!r) return r.error();
  out.attn = std::move(r).value();
  return out;
}

// apply_rope_in_place's position check (microsoft.rs:125-133, :212-230) for
// positions past .. past + S - 1: the first position past the table's end.
Result<Unit, OpError> check_positions(size_t past, size_t S, int32_t rows, size_t B, size_t H) {
  if (B == 0 || H == 0 || S == 0) return Unit{};
  if (past + S > (size_t)rows) {
    const size_t bad = past >= (size_t)rows ? past : (size_t)rows;
    return shape_fmt("apply_rope_in_place: position %lld out of cache range %lld", (long long)bad,
                     (long long)rows);
  }
  return Unit{};
}

}  // namespace

Result<AttentionOutputs, OpError> op_group_query_attention(
    RocmRuntime& runtime, const std::vector<const DeviceTensor*>& inputs, int64_t num_heads,
    int64_t kv_num_heads, std::optional<float> scale_attr, int64_t local_window_size,
    bool do_rotary, bool rotary_interleaved) {
  if (local_window_size != -1)
    return OpError::attribute("GroupQueryAttention: local_window_size != -1 not supported in this tier");
  const DeviceTensor* q = slot(inputs, 0);
  if (!q) return OpError::shape("GroupQueryAttention: missing query");
  const DeviceTensor* k = slot(inputs, 1);
  if (!k) return OpError::shape("GroupQueryAttention: missing key");
  const DeviceTensor* v = slot(inputs, 2);
  if (!v) return OpError::shape("GroupQueryAttention: missing value");
  const DeviceTensor* past_key = slot(inputs, 3);
  const DeviceTensor* past_value = slot(inputs, 4);
  const DeviceTensor* cos = slot(inputs, 7);
  const DeviceTensor* sin = slot(inputs, 8);
  if (q->dtype != DataType::Float || k->dtype != DataType::Float || v->dtype != DataType::Float)
    return OpError::shape("GroupQueryAttention requires Float input");
  if (!q->holds_shape() || !k->holds_shape() || !v->holds_shape())
    return OpError::shape("GroupQueryAttention: input buffer does not hold its shape");
  // gqa_validate (microsoft.rs:933-984) takes rank-3 Q/K/V only
  if (q->shape.size() != 3 || k->shape.size() != 3 || v->shape.size() != 3) {
    if (num_heads <= 0 || kv_num_heads <= 0)
      return OpError::attribute("GroupQueryAttention: num_heads and kv_num_heads must be > 0");
    if (num_heads % kv_num_heads != 0)
      return OpError::attribute("GroupQueryAttention: num_heads must be a multiple of kv_num_heads");
    return OpError::shape("GroupQueryAttention: Q/K/V must be rank-3");
  }
  auto gs = gqa_validate(q->shape, k->shape, v->shape, num_heads, kv_num_heads);
  if (!gs) return gs.error();
  const GqaShape g = gs.value();
  // gqa_past_sk (microsoft.rs:988-1000)
  size_t past = 0;
  if (past_key) {
    if (past_key->shape.size() != 4)
      return OpError::shape("GroupQueryAttention: past_key must be rank-4");
    past = past_key->shape[2] < 0 ? 0 : (size_t)past_key->shape[2];
  }
  RopeTables rope;
  const RopeTables* rope_ptr = nullptr;
  if (do_rotary) {  // gqa_apply_rotary (microsoft.rs:1004-1052)
    if (!cos) return OpError::shape("GroupQueryAttention: do_rotary=1 but cos_cache is missing");
    if (!sin) return OpError::shape("GroupQueryAttention: do_rotary=1 but sin_cache is missing");
    auto rows = check_rope_tables(*cos, *sin, g.head_dim);
    if (!rows) return rows.error();
    auto pc = check_positions(past, g.seq, rows.value(), g.batch, g.num_heads);
    if (!pc) return pc.error();
    rope.cos = (const float*)cos->buffer.as_ptr();
    rope.sin = (const float*)sin->buffer.as_ptr();
    rope.rows = rows.value();
    rope.interleaved = rotary_interleaved;
    rope_ptr = &rope;
  }
  // kv_concat of both pasts (microsoft.rs:1138-1146)
  auto pk = validate_past_kv(past_key, g.batch, g.kv_heads, g.head_dim);
  if (!pk) return pk.error();
  auto pv = validate_past_kv(past_value, g.batch, g.kv_heads, g.head_dim);
  if (!pv) return pv.error();
  if (pk.value() != past || pv.value() != past)
    return OpError::shape("GroupQueryAttention: past_key / past_value sequence mismatch");
  return attention_with_past(runtime, *q, *k, *v, past_key, past_value, past, g, rope_ptr,
                             scale_attr, "ROCm GroupQueryAttention: ");
}

Result<AttentionOutputs, OpError> op_multi_head_attention(
    RocmRuntime& runtime, const std::vector<const DeviceTensor*>& inputs, int64_t num_heads,
    std::optional<float> scale_attr) {
  const DeviceTensor* q = slot(inputs, 0);
  if (!q) return OpError::shape("MultiHeadAttention: missing query");
  const DeviceTensor* k = slot(inputs, 1);
  if (!k) return OpError::shape("MultiHeadAttention: missing key");
  const DeviceTensor* v = slot(inputs, 2);
  if (!v) return OpError::shape("MultiHeadAttention: missing value");
  // inputs 3..5 (bias, key_padding_mask, relative_position_bias) are not read
  const DeviceTensor* past_key = slot(inputs, 6);
  const DeviceTensor* past_value = slot(inputs, 7);
  if (q->dtype != DataType::Float || k->dtype != DataType::Float || v->dtype != DataType::Float)
    return OpError::shape("MultiHeadAttention requires Float input");
  if (!q->holds_shape() || !k->holds_shape() || !v->holds_shape())
    return OpError::shape("MultiHeadAttention: input buffer does not hold its shape");
  if (num_heads <= 0) return OpError::attribute("MultiHeadAttention: num_heads must be > 0");
  if (q->shape.size() != 3 || k->shape.size() != 3 || v->shape.size() != 3)
    return OpError::shape("MultiHeadAttention: Q/K/V must be rank-3 (B, Sq, hidden)");
  const int64_t b = q->shape[0], sq = q->shape[1], hidden = q->shape[2];
  if (b < 0 || sq < 0 || hidden < 0)
    return OpError::shape("MultiHeadAttention: Q/K/V must be rank-3 (B, Sq, hidden)");
  if (hidden % num_heads != 0)
    return OpError::shape("MultiHeadAttention: hidden not divisible by num_heads");
  if (k->shape != q->shape)
    return OpError::shape("MultiHeadAttention: K shape must match Q (unpacked form)");
  if (v->shape != q->shape) return OpError::shape("MultiHeadAttention: V shape must match Q");
  GqaShape g;
  g.num_heads = g.kv_heads = (size_t)num_heads;
  g.batch = (size_t)b;
  g.seq = (size_t)sq;
  g.q_hidden = (size_t)hidden;
  g.head_dim = (size_t)(hidden / num_heads);
  auto pk = validate_past_kv(past_key, g.batch, g.kv_heads, g.head_dim);
  if (!pk) return pk.error();
  auto pv = validate_past_kv(past_value, g.batch, g.kv_heads, g.head_dim);
  if (!pv) return pv.error();
  if (pk.value() != pv.value())
    return OpError::shape("MultiHeadAttention: past_key/past_value sequence length mismatch");
  return attention_with_past(runtime, *q, *k, *v, past_key, past_value, pk.value(), g, nullptr,
                             scale_attr, "ROCm MultiHeadAttention: ");
}

}  // namespace sai::rocm
