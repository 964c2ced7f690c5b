// Tests of the C++ host mirror (smallaios_amd/host/gqa_host.hpp).
//
//   test_gqa_host --cpu        cases that need no device
//   test_gqa_host --gpu        cases that run kernels (one process, device 0)
//   test_gqa_host NAME...      the named cases
//
// The GPU cases restate the reference's own cache and GQA tests
// (onnx-rt/tests/test_cuda.rs:1124-1375 and :3426-3525) for the quantised
// cache, and check a multi-layer prefill + decode session run through
// dispatch_gqa against the oracle (oracle/sai_oracle.h), which this test links
// as the checker. Every case prints PASS/FAIL with its name; the exit status is
// the number of failed cases.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <optional>
#include <random>
#include <string>
#include <tuple>
#include <vector>

#include "../../oracle/sai_oracle.h"
#include "../../smallaios_amd/host/gqa_host.hpp"
#include "../../smallaios_amd/host/gqa_session.hpp"
#include "../../smallaios_amd/host/kv_compression.hpp"

using namespace sai::rocm;

namespace {

struct Failure {
  std::string msg;
};

#define REQUIRE(cond, ...)                                      \
  do {                                                          \
    if (!(cond)) {                                              \
      char _b[512];                                             \
      std::snprintf(_b, sizeof _b, __VA_ARGS__);                \
      throw Failure{std::string(#cond) + ": " + _b};            \
    }                                                           \
  } while (0)

template <class T, class E>
T must(Result<T, E>&& r, const char* what) {
  if (!r) throw Failure{std::string(what) + ": " + r.error().to_string()};
  return std::move(r).value();
}

template <class T>
OpError must_fail(Result<T, OpError>&& r, const char* what) {
  if (r) throw Failure{std::string(what) + ": expected an error"};
  return r.error();
}

template <class T>
SessionError must_fail_session(Result<T, SessionError>&& r, const char* what) {
  if (r) throw Failure{std::string(what) + ": expected an error"};
  return r.error();
}

template <class T>
HipError must_fail_hip(Result<T, HipError>&& r, const char* what) {
  if (r) throw Failure{std::string(what) + ": expected an error"};
  return r.error();
}

std::vector<int64_t> shp(std::initializer_list<int64_t> l) { return std::vector<int64_t>(l); }

// f64 angles rounded to f32: cos/sin [rows, D/2], pairs theta^(-2i/D).
void rope_tables(int rows, int D, double theta, std::vector<float>& c, std::vector<float>& s) {
  c.resize((size_t)rows * D / 2);
  s.resize(c.size());
  for (int p = 0; p < rows; ++p)
    for (int i = 0; i < D / 2; ++i) {
      const double ang = p * std::pow(theta, -2.0 * i / D);
      c[(size_t)p * D / 2 + i] = (float)std::cos(ang);
      s[(size_t)p * D / 2 + i] = (float)std::sin(ang);
    }
}

std::vector<float> gauss(std::mt19937_64& g, size_t n) {
  std::normal_distribution<float> nd(0.0f, 1.0f);
  std::vector<float> v(n);
  for (float& x : v) x = nd(g);
  return v;
}

// The same values as bf16 device bytes and as the f32 values those bytes hold.
DeviceTensor bf16_tensor(std::vector<float>& v, std::vector<int64_t> shape) {
  std::vector<uint16_t> b(v.size());
  for (size_t i = 0; i < v.size(); ++i) {
    b[i] = sai_or_f32_to_bf16(v[i]);
    v[i] = sai_or_bf16_to_f32(b[i]);
  }
  return must(DeviceTensor::from_host(b.data(), b.size() * 2, std::move(shape), DataType::BFloat16),
              "bf16 upload");
}

DeviceTensor f32_tensor(const std::vector<float>& v, std::vector<int64_t> shape) {
  return must(DeviceTensor::from_f32(v, std::move(shape)), "f32 upload");
}

DeviceTensor fill_tensor(size_t heads, size_t d, float fill) {
  return f32_tensor(std::vector<float>(heads * d, fill), shp({1, (int64_t)heads, 1, (int64_t)d}));
}

// |got - want| <= 2e-3 + 1e-2 |want| elementwise (the parity bar for outputs).
void close(const std::vector<float>& got, const std::vector<float>& want, const char* what) {
  REQUIRE(got.size() == want.size(), "%s: %zu vs %zu elements", what, got.size(), want.size());
  for (size_t i = 0; i < got.size(); ++i) {
    const float tol = 2e-3f + 1e-2f * std::fabs(want[i]);
    REQUIRE(std::isfinite(got[i]) && std::fabs(got[i] - want[i]) <= tol,
            "%s: element %zu got %.7g want %.7g", what, i, got[i], want[i]);
  }
}

// A bf16 attention output against the f32 oracle: the same bar widened by
// bf16's round-to-nearest (2^-9 of the value, on both sides).
void close_bf16(const std::vector<float>& got, const std::vector<float>& want, const char* what) {
  REQUIRE(got.size() == want.size(), "%s: %zu vs %zu elements", what, got.size(), want.size());
  for (size_t i = 0; i < got.size(); ++i) {
    const float tol = 2e-3f + (1e-2f + 1.0f / 256.0f) * std::fabs(want[i]);
    REQUIRE(std::isfinite(got[i]) && std::fabs(got[i] - want[i]) <= tol,
            "%s: element %zu got %.7g want %.7g", what, i, got[i], want[i]);
  }
}

// The values of an f32 or bf16 device tensor, as f32.
std::vector<float> host_values(const DeviceTensor& t) {
  if (t.dtype == DataType::Float) return must(t.to_host_f32(), "to_host_f32");
  REQUIRE(t.dtype == DataType::BFloat16, "dtype %d", (int)t.dtype);
  const std::vector<uint8_t> raw = must(t.to_host(), "to_host");
  std::vector<float> v(raw.size() / 2);
  for (size_t i = 0; i < v.size(); ++i) {
    uint16_t b;
    std::memcpy(&b, raw.data() + 2 * i, 2);
    v[i] = sai_or_bf16_to_f32(b);
  }
  return v;
}

// ------------------------------------------------------------- CPU cases ---
void cpu_attrs() {
  GqaAttrs d = parse_gqa_attrs({});
  REQUIRE(d.num_heads == 0 && d.kv_num_heads == 0 && d.local_window_size == -1, "defaults");
  REQUIRE(d.do_rotary && !d.do_rotary_set && !d.rotary_interleaved && !d.scale, "defaults");
  GqaAttrs a = parse_gqa_attrs({AttributeProto::make_int("num_heads", 32),
                                AttributeProto::make_int("kv_num_heads", 8),
                                AttributeProto::make_int("num_heads", 7),  // first one wins
                                AttributeProto::make_float("kv_num_heads", 3.0f),  // wrong type
                                AttributeProto::make_int("do_rotary", 0),
                                AttributeProto::make_int("rotary_interleaved", 5),
                                AttributeProto::make_int("scale", 2),  // wrong type
                                AttributeProto::make_float("scale", 0.125f)});
  REQUIRE(a.num_heads == 32 && a.kv_num_heads == 8, "%lld %lld", (long long)a.num_heads,
          (long long)a.kv_num_heads);
  REQUIRE(!a.do_rotary && a.do_rotary_set && a.rotary_interleaved, "rotary flags");
  REQUIRE(a.scale && *a.scale == 0.125f, "scale");
}

void cpu_validate() {
  struct Case {
    std::vector<int64_t> q, k, v;
    int64_t nh, kvh;
    OpError::Kind kind;
    const char* msg;
  };
  const Case cases[] = {
      {shp({1, 1, 64}), shp({1, 1, 32}), shp({1, 1, 32}), 0, 1, OpError::Kind::InvalidAttribute,
       "GroupQueryAttention: num_heads and kv_num_heads must be > 0"},
      {shp({1, 1, 64}), shp({1, 1, 32}), shp({1, 1, 32}), 3, 2, OpError::Kind::InvalidAttribute,
       "GroupQueryAttention: num_heads must be a multiple of kv_num_heads"},
      {shp({1, 64}), shp({1, 1, 32}), shp({1, 1, 32}), 2, 1, OpError::Kind::ShapeMismatch,
       "GroupQueryAttention: Q/K/V must be rank-3"},
      {shp({1, 1, 65}), shp({1, 1, 32}), shp({1, 1, 32}), 2, 1, OpError::Kind::ShapeMismatch,
       "GroupQueryAttention: q_hidden not divisible by num_heads"},
      {shp({1, 1, 64}), shp({1, 1, 33}), shp({1, 1, 33}), 4, 2, OpError::Kind::ShapeMismatch,
       "GroupQueryAttention: kv_hidden not divisible by kv_num_heads"},
      {shp({1, 1, 64}), shp({1, 1, 64}), shp({1, 1, 64}), 2, 1, OpError::Kind::ShapeMismatch,
       "GroupQueryAttention: Q and KV head_dim must match"},
      {shp({1, 1, 64}), shp({1, 1, 32}), shp({1, 1, 16}), 2, 1, OpError::Kind::ShapeMismatch,
       "GroupQueryAttention: key and value must have the same shape"},
  };
  for (const Case& c : cases) {
    OpError e = must_fail(gqa_validate(c.q, c.k, c.v, c.nh, c.kvh), c.msg);
    REQUIRE(e.kind == c.kind && e.message == c.msg, "got '%s'", e.to_string().c_str());
  }
  GqaShape g = must(gqa_validate(shp({2, 5, 4096}), shp({2, 5, 1024}), shp({2, 5, 1024}), 32, 8),
                    "valid rank-3");
  REQUIRE(g.num_heads == 32 && g.kv_heads == 8 && g.batch == 2 && g.seq == 5 && g.head_dim == 128,
          "rank-3 shape facts");
  // rank-4 [B, H, 1, D]: heads from the shapes, attributes ignored
  g = must(gqa_validate(shp({1, 8, 1, 64}), shp({1, 2, 1, 64}), shp({1, 2, 1, 64}), 0, 0),
           "valid rank-4");
  REQUIRE(g.num_heads == 8 && g.kv_heads == 2 && g.seq == 1 && g.head_dim == 64, "rank-4 facts");
  OpError e = must_fail(gqa_validate(shp({1, 8, 3, 64}), shp({1, 2, 3, 64}), shp({1, 2, 3, 64}), 0, 0),
                        "rank-4 S > 1");
  REQUIRE(e.kind == OpError::Kind::ShapeMismatch, "rank-4 S>1 kind");
}

void cpu_errors_and_types() {
  REQUIRE(OpError::shape("x").to_string() == "shape mismatch: x", "display");
  REQUIRE(OpError::attribute("x").to_string() == "invalid attribute: x", "display");
  REQUIRE(OpError::unsupported("x").to_string() == "unsupported operator: x", "display");
  REQUIRE(OpError::internal("x").to_string() == "internal error: x", "display");
  REQUIRE(HipError::runtime("kv_cache_append:layer_idx").to_string() ==
              "HIP kv_cache_append:layer_idx failed: code -1",
          "%s", HipError::runtime("kv_cache_append:layer_idx").to_string().c_str());
  REQUIRE(HipError::alloc_failed(64, 2).to_string() == "hipMalloc(64 bytes) failed: code 2", "display");
  REQUIRE(RocmRuntime::supports_op("GroupQueryAttention"), "supports GQA");
  REQUIRE(RocmRuntime::supports_op("RotaryEmbedding"), "supports RotaryEmbedding");
  REQUIRE(!RocmRuntime::supports_op("MatMul") && !RocmRuntime::supports_op(""),
          "only GQA and RotaryEmbedding");
  REQUIRE(element_size(DataType::Float) == 4 && element_size(DataType::BFloat16) == 2 &&
              element_size(DataType::Int64) == 8 && element_size(DataType::Int8) == 1,
          "element sizes");
  DeviceTensor t;
  t.shape = shp({2, -1, 3});
  REQUIRE(t.total_elements() == 0 && t.byte_size() == 0, "negative dim");
  t.shape = shp({2, 3, 4});
  t.dtype = DataType::BFloat16;
  REQUIRE(t.total_elements() == 24 && t.byte_size() == 48, "sizes");
  // a shape with no buffer behind it is rejected by every entry point
  REQUIRE(!t.holds_shape(), "shape without a buffer");
  t.shape = shp({2, 0, 4});
  REQUIRE(t.holds_shape(), "empty shape needs no buffer");
  HipError e = must_fail_hip(RocmRuntime::init(1 << 20), "device out of range");
  REQUIRE(e.kind == HipError::Kind::NoDevice, "%s", e.to_string().c_str());
}

// ------------------------------------------------------------- GPU cases ---
RocmRuntime& runtime() {
  static RocmRuntime rt = must(RocmRuntime::init(0), "RocmRuntime::init");
  return rt;
}

// test_cuda.rs:1124 (test_kv_cache_allocate_and_append), per quantisation.
void gpu_cache_allocate_and_append() {
  for (KvQuant quant : {KvQuant::Int8, KvQuant::Int4}) {
    const size_t L = 4, H = 8, D = 128, S = 16;
    GpuKvCache cache = must(GpuKvCache::allocate(runtime(), L, H, D, S, quant,
                                                 std::vector<LayerKind>(L, LayerKind::global())),
                            "allocate");
    REQUIRE(cache.num_layers() == L && cache.current_position() == 0 && cache.max_seq_len() == S,
            "geometry");
    KvView v0 = must(cache.view(0), "empty view");
    REQUIRE(v0.token_count == 0 && v0.pool && v0.block_bytes > 0, "empty view");
    for (size_t l = 0; l < L; ++l) {
      const float fill = (float)(l + 1) * 0.25f;
      DeviceTensor k = fill_tensor(H, D, fill), v = fill_tensor(H, D, fill + 0.5f);
      must(cache.append(l, k, v), "append");
    }
    REQUIRE(cache.pending() == 1, "pending after append");
    must(cache.advance_position(), "advance_position");
    REQUIRE(cache.current_position() == 1 && cache.pending() == 0, "position 1");
    for (size_t l = 0; l < L; ++l) {
      KvView view = must(cache.view(l), "view");
      REQUIRE(view.token_count == 1 && view.num_kv_heads == H && view.head_dim == D &&
                  view.quant == quant,
              "view fields");
      const float ek = (float)(l + 1) * 0.25f, ev = ek + 0.5f;
      for (size_t h = 0; h < H; ++h) {
        auto kv = must(cache.read_dequantized(l, 0, h, 0, 1), "read");
        for (size_t d = 0; d < D; ++d) {
          REQUIRE(std::fabs(kv.first[d] - ek) < 1e-3f, "layer %zu k %g != %g", l, kv.first[d], ek);
          REQUIRE(std::fabs(kv.second[d] - ev) < 1e-3f, "layer %zu v %g != %g", l, kv.second[d], ev);
        }
      }
    }
  }
}

// test_cuda.rs:1203 (test_kv_cache_multiple_tokens), D = 64.
void gpu_cache_multiple_tokens() {
  const size_t L = 2, H = 4, D = 64, S = 8;
  GpuKvCache cache = must(GpuKvCache::allocate(runtime(), L, H, D, S, KvQuant::Int8,
                                               std::vector<LayerKind>(L, LayerKind::global())),
                          "allocate");
  for (size_t pos = 0; pos < 3; ++pos) {
    for (size_t l = 0; l < L; ++l) {
      DeviceTensor k = fill_tensor(H, D, (float)(pos + 1) * 0.125f);
      DeviceTensor v = fill_tensor(H, D, (float)(pos + 1) * 0.25f);
      must(cache.append(l, k, v), "append");
    }
    must(cache.advance_position(), "advance");
  }
  REQUIRE(cache.current_position() == 3, "position");
  for (size_t l = 0; l < L; ++l) {
    REQUIRE(must(cache.view(l), "view").token_count == 3, "token count");
    for (size_t h = 0; h < H; ++h) {
      auto kv = must(cache.read_dequantized(l, 0, h, 0, 3), "read");
      for (size_t pos = 0; pos < 3; ++pos)
        for (size_t d = 0; d < D; ++d) {
          REQUIRE(std::fabs(kv.first[pos * D + d] - (float)(pos + 1) * 0.125f) < 1e-3f, "k pos %zu", pos);
          REQUIRE(std::fabs(kv.second[pos * D + d] - (float)(pos + 1) * 0.25f) < 1e-3f, "v pos %zu", pos);
        }
    }
  }
}

// test_cuda.rs:1339 (test_kv_cache_reset), D = 64.
void gpu_cache_reset() {
  const size_t H = 2, D = 64, S = 8;
  GpuKvCache cache = must(GpuKvCache::allocate(runtime(), 1, H, D, S, KvQuant::Int8,
                                               {LayerKind::global()}),
                          "allocate");
  for (size_t pos = 0; pos < 2; ++pos) {
    DeviceTensor k = fill_tensor(H, D, (float)(pos + 1) * 0.5f);
    must(cache.append(0, k, k), "append");
    must(cache.advance_position(), "advance");
  }
  REQUIRE(cache.current_position() == 2, "position 2");
  cache.reset();
  REQUIRE(cache.current_position() == 0 && must(cache.view(0), "view").token_count == 0, "reset");
  DeviceTensor k = fill_tensor(H, D, 9.0f);
  must(cache.append(0, k, k), "append after reset");
  must(cache.advance_position(), "advance");
  auto kv = must(cache.read_dequantized(0, 0, 1, 0, 1), "read slot 0");
  for (size_t d = 0; d < D; ++d) REQUIRE(std::fabs(kv.first[d] - 9.0f) < 1e-3f, "slot 0 %g", kv.first[d]);
}

// The cache's error contract (kv_cache.rs:129-300 error sites).
void gpu_cache_errors() {
  auto op_of = [](const HipError& e) { return e.op; };
  RocmRuntime& rt = runtime();
  REQUIRE(op_of(must_fail_hip(GpuKvCache::allocate(rt, 2, 2, 64, 8, KvQuant::Int8, {LayerKind::global()}),
                              "kinds")) == "kv_cache_allocate:layer_kinds_len", "layer_kinds_len");
  REQUIRE(op_of(must_fail_hip(GpuKvCache::allocate(rt, 1, 0, 64, 8, KvQuant::Int8, {LayerKind::global()}),
                              "zero")) == "kv_cache_allocate:zero_dim", "zero_dim");
  REQUIRE(op_of(must_fail_hip(GpuKvCache::allocate(rt, 1, 2, 64, 8, KvQuant::Int8,
                                                   {LayerKind::sliding_window(0)}),
                              "window")) == "kv_cache_allocate:sliding_window", "sliding_window 0");
  REQUIRE(op_of(must_fail_hip(GpuKvCache::allocate(rt, 1, 2, 16, 8, KvQuant::Int8, {LayerKind::global()}),
                              "head_dim")) == "kv_cache_allocate:unsupported_head_dim", "head_dim");
  // int4's groups of 32 do not divide 168 (int8 takes it)
  REQUIRE(op_of(must_fail_hip(GpuKvCache::allocate(rt, 1, 2, 168, 8, KvQuant::Int4, {LayerKind::global()}),
                              "int4 168")) == "kv_cache_allocate:unsupported_head_dim", "int4 head_dim 168");
  GpuKvCache cache = must(GpuKvCache::allocate(rt, 1, 2, 64, 2, KvQuant::Int8, {LayerKind::global()}),
                          "allocate");
  DeviceTensor k = fill_tensor(2, 64, 1.0f);
  REQUIRE(op_of(must_fail_hip(cache.append(1, k, k), "layer")) == "kv_cache_append:layer_idx", "layer_idx");
  DeviceTensor bad = fill_tensor(2, 32, 1.0f);
  REQUIRE(op_of(must_fail_hip(cache.append(0, bad, bad), "size")) ==
              "kv_cache_append:tensor_byte_size_mismatch", "byte size");
  DeviceTensor ints = must(DeviceTensor::alloc(shp({1, 2, 1, 64}), DataType::Int32), "alloc");
  REQUIRE(op_of(must_fail_hip(cache.append(0, ints, ints), "dtype")) == "kv_cache_append:dtype_mismatch",
          "dtype");
  REQUIRE(op_of(must_fail_hip(cache.advance_position(), "nothing")) == "kv_cache_advance:nothing_pending",
          "nothing pending");
  REQUIRE(op_of(must_fail_hip(cache.view(3), "view")) == "kv_cache_view:layer_idx", "view layer");
  REQUIRE(op_of(must_fail_hip(cache.view_pending(3), "view")) == "kv_cache_view_pending:layer_idx",
          "view_pending layer");
  for (int i = 0; i < 2; ++i) {
    must(cache.append(0, k, k), "append");
    REQUIRE(must(cache.view_pending(0), "view_pending").token_count == (size_t)i + 1, "pending view");
    must(cache.advance_position(), "advance");
  }
  REQUIRE(op_of(must_fail_hip(cache.append(0, k, k), "overflow")) == "kv_cache_append:position_overflow",
          "position_overflow");
  // batch switch only at position 0
  DeviceTensor k2 = f32_tensor(std::vector<float>(2 * 2 * 64, 1.0f), shp({2, 1, 128}));
  REQUIRE(op_of(must_fail_hip(cache.append(0, k2, k2), "batch")) == "kv_cache_append:batch_mismatch",
          "batch beyond max_batch");
}

// test_cuda.rs:3464 (test_gpu_gqa_with_cache_first_token): one token through
// the cache path; the output is that token's (dequantised) V.
void gpu_gqa_with_cache_first_token() {
  const size_t h = 2, hd = 64, max_seq = 8;
  std::vector<float> q(h * hd), k(h * hd), v(h * hd);
  for (size_t i = 0; i < h * hd; ++i) {
    q[i] = (float)i * 0.1f;
    k[i] = std::sin((float)i * 0.03f);
    v[i] = (float)i * 0.05f + 1.0f;
  }
  const auto s4 = shp({1, (int64_t)h, 1, (int64_t)hd});
  DeviceTensor dq = f32_tensor(q, s4), dk = f32_tensor(k, s4), dv = f32_tensor(v, s4);
  GpuKvCache cache = must(GpuKvCache::allocate(runtime(), 1, h, hd, max_seq, KvQuant::Int8,
                                               {LayerKind::global()}),
                          "alloc cache");
  KvCacheDispatchCtx ctx{&cache, 0};
  auto outs = must(dispatch_gqa(runtime(), {&dq, &dk, &dv}, {}, &ctx), "dispatch_gqa");
  REQUIRE(ctx.next_layer_idx == 1, "layer counter");
  must(cache.advance_position(), "advance_position");
  REQUIRE(cache.current_position() == 1, "cache should hold one token");
  REQUIRE(outs.size() == 1 && outs[0].shape == shp({1, 1, (int64_t)(h * hd)}), "output shape");
  std::vector<float> got = must(outs[0].to_host_f32(), "download");
  for (size_t hh = 0; hh < h; ++hh) {
    auto kv = must(cache.read_dequantized(0, 0, hh, 0, 1), "read");
    std::vector<float> want(kv.second), g(got.begin() + hh * hd, got.begin() + (hh + 1) * hd);
    close(g, want, "first token = dequantised V");
    float amax = 0;
    for (size_t d = 0; d < hd; ++d) amax = std::max(amax, std::fabs(v[hh * hd + d]));
    for (size_t d = 0; d < hd; ++d)
      REQUIRE(std::fabs(want[d] - v[hh * hd + d]) <= amax / 254.0f * 1.0001f, "quantisation bound");
  }
}

// test_cuda.rs:3426 (test_gpu_gqa_first_token_no_history): no cache context.
void gpu_gqa_first_token_no_history() {
  const size_t h = 2, hd = 128;
  std::vector<float> q(h * hd), k(h * hd, 0.0f), v(h * hd);
  for (size_t i = 0; i < h * hd; ++i) {
    q[i] = (float)i * 0.1f;
    v[i] = (float)i * 0.05f + 1.0f;
  }
  const auto s3q = shp({1, 1, (int64_t)(h * hd)});
  DeviceTensor dq = f32_tensor(q, s3q), dk = f32_tensor(k, s3q), dv = f32_tensor(v, s3q);
  const std::vector<AttributeProto> attrs = {AttributeProto::make_int("num_heads", (int64_t)h),
                                             AttributeProto::make_int("kv_num_heads", (int64_t)h)};
  auto outs = must(dispatch_gqa(runtime(), {&dq, &dk, &dv}, attrs, nullptr), "dispatch_gqa");
  REQUIRE(outs[0].shape == s3q, "output shape");
  std::vector<float> got = must(outs[0].to_host_f32(), "download");
  for (size_t hh = 0; hh < h; ++hh) {
    float amax = 0;
    for (size_t d = 0; d < hd; ++d) amax = std::max(amax, std::fabs(v[hh * hd + d]));
    for (size_t d = 0; d < hd; ++d) {
      const float want = v[hh * hd + d];
      REQUIRE(std::fabs(got[hh * hd + d] - want) <= amax / 254.0f + 2e-3f + 1e-2f * std::fabs(want),
              "h=%zu d=%zu got %g want %g", hh, d, got[hh * hd + d], want);
    }
  }
}

// dispatch_gqa's error contract.
void gpu_dispatch_errors() {
  RocmRuntime& rt = runtime();
  const auto s3 = shp({1, 1, 256}), s3kv = shp({1, 1, 128});
  DeviceTensor q = f32_tensor(std::vector<float>(256, 0.5f), s3);
  DeviceTensor k = f32_tensor(std::vector<float>(128, 0.5f), s3kv);
  const std::vector<AttributeProto> heads = {AttributeProto::make_int("num_heads", 4),
                                             AttributeProto::make_int("kv_num_heads", 2)};
  auto expect = [&](Result<std::vector<DeviceTensor>, OpError>&& r, OpError::Kind kind,
                    const std::string& msg, const char* what) {
    OpError e = must_fail(std::move(r), what);
    REQUIRE(e.kind == kind && e.message.find(msg) != std::string::npos, "%s: got '%s'", what,
            e.to_string().c_str());
  };
  expect(dispatch_gqa(rt, {&q, nullptr, &k}, heads, nullptr), OpError::Kind::InternalError,
         "GPU GroupQueryAttention: missing input 'K'", "missing K");
  expect(dispatch_gqa(rt, {&q, &k, &k}, {}, nullptr), OpError::Kind::InvalidAttribute,
         "num_heads and kv_num_heads must be > 0", "rank-3 without heads");
  std::vector<AttributeProto> rot = heads;
  rot.push_back(AttributeProto::make_int("do_rotary", 1));
  expect(dispatch_gqa(rt, {&q, &k, &k}, rot, nullptr), OpError::Kind::ShapeMismatch,
         "do_rotary=1 but cos_cache is missing", "explicit do_rotary without cos");
  DeviceTensor cs = f32_tensor(std::vector<float>(8 * 32, 1.0f), shp({8, 32}));
  expect(dispatch_gqa(rt, {&q, &k, &k, nullptr, nullptr, nullptr, nullptr, &cs, nullptr}, heads,
                      nullptr),
         OpError::Kind::ShapeMismatch, "do_rotary=1 but sin_cache is missing", "cos without sin");
  // a tensor whose shape claims more than its buffer holds
  DeviceTensor short_k = f32_tensor(std::vector<float>(64, 0.5f), shp({1, 1, 64}));
  short_k.shape = s3kv;
  expect(dispatch_gqa(rt, {&q, &short_k, &k}, heads, nullptr), OpError::Kind::ShapeMismatch,
         "input buffer does not hold its shape", "K buffer shorter than its shape");
  DeviceTensor short_q = f32_tensor(std::vector<float>(128, 0.5f), shp({1, 1, 128}));
  short_q.shape = s3;
  expect(dispatch_gqa(rt, {&short_q, &k, &k}, heads, nullptr), OpError::Kind::ShapeMismatch,
         "input buffer does not hold its shape", "Q buffer shorter than its shape");
  OpError eo = must_fail(op_group_query_attention(rt, {&short_q, &k, &k}, 4, 2, std::nullopt, -1,
                                                  false, false),
                         "CPU-op Q buffer shorter than its shape");
  REQUIRE(eo.kind == OpError::Kind::ShapeMismatch &&
              eo.message.find("does not hold its shape") != std::string::npos,
          "%s", eo.to_string().c_str());
  DeviceTensor short_cs = f32_tensor(std::vector<float>(16, 1.0f), shp({1, 16}));
  short_cs.shape = shp({8, 32});
  expect(dispatch_gqa(rt, {&q, &k, &k, nullptr, nullptr, nullptr, nullptr, &short_cs, &cs}, heads,
                      nullptr),
         OpError::Kind::ShapeMismatch, "cos/sin buffer does not hold its shape",
         "cos buffer shorter than its shape");
  GpuKvCache cache = must(GpuKvCache::allocate(rt, 1, 2, 64, 32, KvQuant::Int8,
                                               std::vector<LayerKind>(1, LayerKind::global())),
                          "cache");
  HipError he = must_fail_hip(cache.append(0, short_k, k, nullptr), "append short K");
  REQUIRE(he.to_string().find("tensor_byte_size_mismatch") != std::string::npos, "%s",
          he.to_string().c_str());
}

}  // namespace

// RoPE table checks (validate_rope_caches, ops/microsoft.rs:71-110), the
// kernels' group sizes, and a cache whose geometry differs from the node's.
static void gpu_dispatch_rope_tables() {
  RocmRuntime& rt = runtime();
  DeviceTensor q = f32_tensor(std::vector<float>(256, 0.5f), shp({1, 1, 256}));
  DeviceTensor k = f32_tensor(std::vector<float>(128, 0.5f), shp({1, 1, 128}));
  const std::vector<AttributeProto> heads = {AttributeProto::make_int("num_heads", 4),
                                             AttributeProto::make_int("kv_num_heads", 2)};
  DeviceTensor bad = f32_tensor(std::vector<float>(8 * 16, 1.0f), shp({8, 16}));
  OpError e = must_fail(
      dispatch_gqa(rt, {&q, &k, &k, nullptr, nullptr, nullptr, nullptr, &bad, &bad}, heads, nullptr),
      "inner dim 16");
  REQUIRE(e.kind == OpError::Kind::ShapeMismatch &&
              e.message == "apply_rope_in_place: cache inner dim 16 != rotary_dim/2 = 32",
          "got '%s'", e.to_string().c_str());
  DeviceTensor ok = f32_tensor(std::vector<float>(8 * 32, 1.0f), shp({8, 32}));
  DeviceTensor r2 = f32_tensor(std::vector<float>(8 * 32, 1.0f), shp({8, 32}));
  DeviceTensor i32 = must(DeviceTensor::alloc(shp({8, 32}), DataType::Int32), "alloc");
  e = must_fail(dispatch_gqa(rt, {&q, &k, &k, nullptr, nullptr, nullptr, nullptr, &i32, &r2}, heads,
                             nullptr),
                "int tables");
  REQUIRE(e.message == "RotaryEmbedding requires Float input", "got '%s'", e.to_string().c_str());
  // group of 3 query heads per KV head: not a kernel shape
  DeviceTensor q6 = f32_tensor(std::vector<float>(384, 0.5f), shp({1, 1, 384}));
  e = must_fail(dispatch_gqa(rt, {&q6, &k, &k},
                             {AttributeProto::make_int("num_heads", 6),
                              AttributeProto::make_int("kv_num_heads", 2)},
                             nullptr),
                "group 3");
  REQUIRE(e.kind == OpError::Kind::UnsupportedOp, "got '%s'", e.to_string().c_str());
  // a correct table set runs
  auto outs = must(dispatch_gqa(rt, {&q, &k, &k, nullptr, nullptr, nullptr, nullptr, &ok, &r2},
                                heads, nullptr),
                   "valid tables");
  REQUIRE(outs[0].shape == shp({1, 1, 256}), "shape");
  // a cache whose geometry differs from the node's
  GpuKvCache cache = must(GpuKvCache::allocate(rt, 1, 4, 64, 8, KvQuant::Int8, {LayerKind::global()}),
                          "allocate");
  KvCacheDispatchCtx ctx{&cache, 0};
  e = must_fail(dispatch_gqa(rt, {&q, &k, &k}, heads, &ctx), "geometry");
  REQUIRE(e.kind == OpError::Kind::ShapeMismatch && ctx.next_layer_idx == 1,
          "got '%s', layer %zu", e.to_string().c_str(), ctx.next_layer_idx);
}

// A session: `layers` GQA nodes per forward pass over one cache, a prefill
// chunk of `prefill` tokens then `steps` decode passes, each pass
// followed by one advance_position. Every node's output and the cache
// contents are checked against the oracle: the oracle quantises the same
// ------------------------------------------------------- RotaryEmbedding ---
// make_rope_caches with taylor_cos / taylor_sin (ops/microsoft.rs:1318-1343),
// f32 throughout like the Rust test helpers.
float taylor_cos(float x) {
  const float x2 = x * x;
  return 1.0f - x2 / 2.0f + x2 * x2 / 24.0f - x2 * x2 * x2 / 720.0f;
}
float taylor_sin(float x) {
  const float x2 = x * x;
  return x * (1.0f - x2 / 6.0f + x2 * x2 / 120.0f - x2 * x2 * x2 / 5040.0f);
}
std::pair<DeviceTensor, DeviceTensor> make_rope_caches(int max_seq, int half) {
  std::vector<float> c, s;
  for (int p = 0; p < max_seq; ++p)
    for (int i = 0; i < half; ++i) {
      const float theta = (float)p * (0.1f + (float)i * 0.01f);
      c.push_back(taylor_cos(theta));
      s.push_back(taylor_sin(theta));
    }
  return {f32_tensor(c, shp({max_seq, half})), f32_tensor(s, shp({max_seq, half}))};
}

DeviceTensor i64_tensor(const std::vector<int64_t>& v, std::vector<int64_t> shape) {
  return must(DeviceTensor::from_host(v.data(), v.size() * 8, std::move(shape), DataType::Int64),
              "i64 upload");
}

std::vector<float> host_f32(const DeviceTensor& t) { return must(t.to_host_f32(), "to_host_f32"); }

// The reference's microsoft.rs RotaryEmbedding tests (:1346-1416, :1876-1939)
// through op_rotary_embedding, plus its rank-3 view and partial rotation
// against the oracle.
void gpu_rotary_cpu_op_kats() {
  RocmRuntime& rt = runtime();
  const std::vector<float> x4 = {1.0f, 2.0f, 3.0f, 4.0f};
  {  // rope_position_zero_is_identity / rope_interleaved_position_zero_identity
    auto [c, s] = make_rope_caches(4, 2);
    DeviceTensor in = f32_tensor(x4, shp({1, 1, 1, 4}));
    DeviceTensor pos = i64_tensor({0}, shp({1, 1}));
    for (bool il : {false, true}) {
      DeviceTensor out = must(op_rotary_embedding(rt, {&in, &pos, &c, &s}, il, 0, 1), "pos 0");
      const std::vector<float> v = host_f32(out);
      for (int i = 0; i < 4; ++i) REQUIRE(std::fabs(v[i] - x4[i]) < 1e-5f, "identity %d", i);
    }
  }
  {  // rope_interleaved_vs_noninterleaved_differ
    auto [c, s] = make_rope_caches(4, 2);
    DeviceTensor in = f32_tensor(x4, shp({1, 1, 1, 4}));
    DeviceTensor pos = i64_tensor({1}, shp({1, 1}));
    const std::vector<float> a = host_f32(must(op_rotary_embedding(rt, {&in, &pos, &c, &s}, false, 0, 1), "a"));
    const std::vector<float> b = host_f32(must(op_rotary_embedding(rt, {&in, &pos, &c, &s}, true, 0, 1), "b"));
    bool diff = false;
    for (int i = 0; i < 4; ++i) diff |= std::fabs(a[i] - b[i]) > 1e-4f;
    REQUIRE(diff, "interleaved and non-interleaved RoPE should differ");
  }
  {  // rope_non_interleaved_manual_calc
    auto [c, s] = make_rope_caches(2, 2);
    DeviceTensor in = f32_tensor(x4, shp({1, 1, 1, 4}));
    DeviceTensor pos = i64_tensor({1}, shp({1, 1}));
    const std::vector<float> v = host_f32(must(op_rotary_embedding(rt, {&in, &pos, &c, &s}, false, 0, 1), "manual"));
    const float c0 = taylor_cos(0.1f), s0 = taylor_sin(0.1f), c1 = taylor_cos(0.11f), s1 = taylor_sin(0.11f);
    const float e[4] = {c0 * 1.0f - s0 * 3.0f, c1 * 2.0f - s1 * 4.0f, s0 * 1.0f + c0 * 3.0f,
                        s1 * 2.0f + c1 * 4.0f};
    for (int i = 0; i < 4; ++i) REQUIRE(std::fabs(v[i] - e[i]) < 1e-4f, "manual %d: %g vs %g", i, v[i], e[i]);
  }
  {  // rope_int32_positions
    auto [c, s] = make_rope_caches(4, 2);
    DeviceTensor in = f32_tensor(x4, shp({1, 1, 1, 4}));
    const int32_t zero = 0;
    DeviceTensor pos = must(DeviceTensor::from_host(&zero, 4, shp({1, 1}), DataType::Int32), "i32");
    const std::vector<float> v = host_f32(must(op_rotary_embedding(rt, {&in, &pos, &c, &s}, false, 0, 1), "i32 pos"));
    for (int i = 0; i < 4; ++i) REQUIRE(std::fabs(v[i] - x4[i]) < 1e-5f, "i32 identity %d", i);
  }
  {  // rope_rank3_reshape_path
    auto [c, s] = make_rope_caches(4, 1);
    DeviceTensor in = f32_tensor(x4, shp({1, 1, 4}));
    DeviceTensor pos = i64_tensor({0}, shp({1, 1}));
    DeviceTensor out = must(op_rotary_embedding(rt, {&in, &pos, &c, &s}, false, 0, 2), "rank3");
    REQUIRE(out.shape == shp({1, 1, 4}), "rank-3 output shape");
  }
  {  // rope_rejects_bad_rank / _bad_num_heads_for_rank3 / _missing_inputs
    auto [c, s] = make_rope_caches(2, 2);
    DeviceTensor r2 = f32_tensor(x4, shp({1, 4}));
    DeviceTensor r3 = f32_tensor(x4, shp({1, 1, 4}));
    DeviceTensor r4 = f32_tensor(x4, shp({1, 1, 1, 4}));
    DeviceTensor pos = i64_tensor({0}, shp({1}));
    OpError e = must_fail(op_rotary_embedding(rt, {&r2, &pos, &c, &s}, false, 0, 1), "rank 2");
    REQUIRE(e.kind == OpError::Kind::ShapeMismatch &&
                e.message == "RotaryEmbedding: input must be rank-3 or rank-4", "%s", e.to_string().c_str());
    e = must_fail(op_rotary_embedding(rt, {&r3, &pos, &c, &s}, false, 0, 0), "num_heads 0");
    REQUIRE(e.kind == OpError::Kind::InvalidAttribute &&
                e.message == "RotaryEmbedding: num_heads must be > 0 for rank-3 input", "%s", e.to_string().c_str());
    e = must_fail(op_rotary_embedding(rt, {&r4}, false, 0, 1), "missing");
    REQUIRE(e.message == "RotaryEmbedding: missing position_ids", "%s", e.to_string().c_str());
    e = must_fail(op_rotary_embedding(rt, {&r4, &pos, &c}, false, 0, 1), "missing sin");
    REQUIRE(e.message == "RotaryEmbedding: missing sin_cache", "%s", e.to_string().c_str());
    DeviceTensor pos9 = i64_tensor({9}, shp({1}));
    e = must_fail(op_rotary_embedding(rt, {&r4, &pos9, &c, &s}, false, 0, 1), "pos 9");
    REQUIRE(e.kind == OpError::Kind::ShapeMismatch &&
                e.message == "apply_rope_in_place: position 9 out of cache range 2", "%s", e.to_string().c_str());
    DeviceTensor pos2 = i64_tensor({0, 1}, shp({2}));
    e = must_fail(op_rotary_embedding(rt, {&r4, &pos2, &c, &s}, false, 0, 1), "n_pos");
    REQUIRE(e.message == "apply_rope_in_place: position_ids length 2 != B*Sq = 1", "%s", e.to_string().c_str());
    e = must_fail(op_rotary_embedding(rt, {&r4, &pos, &c, &s}, false, 3, 1), "odd rotary_dim");
    REQUIRE(e.kind == OpError::Kind::InvalidAttribute &&
                e.message == "apply_rope_in_place: rotary_dim must be even", "%s", e.to_string().c_str());
    e = must_fail(op_rotary_embedding(rt, {&r4, &pos, &c, &s}, false, 2, 1), "cols");
    REQUIRE(e.message == "apply_rope_in_place: cache inner dim 2 != rotary_dim/2 = 1", "%s", e.to_string().c_str());
    DeviceTensor f = i64_tensor({0}, shp({1}));
    f.dtype = DataType::Float16;
    f.shape = shp({4});
    e = must_fail(op_rotary_embedding(rt, {&r4, &f, &c, &s}, false, 0, 1), "pos dtype");
    REQUIRE(e.message == "RotaryEmbedding: position_ids must be int32 or int64", "%s", e.to_string().c_str());
  }
  {  // rank 3 [B, S, H*D] read as [B, H, S, D] over the same bytes; partial rotary_dim
    const int B = 2, S = 3, H = 2, D = 16, RD = 8, rows = 16;
    std::mt19937_64 g(21);
    std::vector<float> x = gauss(g, (size_t)B * S * H * D);
    std::vector<float> c, sn;
    rope_tables(rows, RD, 1e4, c, sn);
    DeviceTensor cd = f32_tensor(c, shp({rows, RD / 2})), sd = f32_tensor(sn, shp({rows, RD / 2}));
    std::vector<int64_t> ids = {5, 2, 9, 0, 1, 15};
    DeviceTensor in = f32_tensor(x, shp({B, S, H * D}));
    DeviceTensor pos = i64_tensor(ids, shp({B, S}));
    for (bool il : {false, true}) {
      const std::vector<float> got = host_f32(must(op_rotary_embedding(rt, {&in, &pos, &cd, &sd}, il, RD, H), "rank3 partial"));
      std::vector<float> want = x;
      REQUIRE(sai_or_apply_rope(want.data(), B, H, S, D, c.data(), sn.data(), rows, RD / 2, ids.data(),
                                (int)ids.size(), il ? 1 : 0, RD) == 0, "oracle");
      REQUIRE(std::memcmp(got.data(), want.data(), got.size() * 4) == 0, "rank-3 partial (il %d) differs from the oracle", (int)il);
    }
  }
}

// The reference's GPU rotary tests (tests/test_cuda.rs:2622-2830) through
// dispatch_rotary_embedding, and the dispatcher's position / layout rules.
void gpu_rotary_dispatch() {
  RocmRuntime& rt = runtime();
  std::mt19937_64 g(33);
  auto check = [&](const std::vector<float>& x, int B, int H, int S, int D, bool bshd,
                   const std::vector<float>& c, const std::vector<float>& sn, int rows, int start,
                   bool il, const std::vector<float>& got, const char* what) {
    // oracle over [B, H, S, D]
    std::vector<float> v((size_t)B * H * S * D);
    for (int b = 0; b < B; ++b)
      for (int h = 0; h < H; ++h)
        for (int s = 0; s < S; ++s)
          for (int d = 0; d < D; ++d) {
            const size_t src = bshd ? (((size_t)b * S + s) * H + h) * D + d : (((size_t)b * H + h) * S + s) * D + d;
            v[(((size_t)b * H + h) * S + s) * D + d] = x[src];
          }
    std::vector<int64_t> ids(S);
    for (int s = 0; s < S; ++s) ids[s] = start + s;
    REQUIRE(sai_or_apply_rope(v.data(), B, H, S, D, c.data(), sn.data(), rows, D / 2, ids.data(), S,
                              il ? 1 : 0, D) == 0, "%s: oracle", what);
    for (int b = 0; b < B; ++b)
      for (int h = 0; h < H; ++h)
        for (int s = 0; s < S; ++s)
          for (int d = 0; d < D; ++d) {
            const size_t dst = bshd ? (((size_t)b * S + s) * H + h) * D + d : (((size_t)b * H + h) * S + s) * D + d;
            const float w = v[(((size_t)b * H + h) * S + s) * D + d];
            REQUIRE(std::memcmp(&got[dst], &w, 4) == 0, "%s: (%d,%d,%d,%d) got %g want %g", what, b, h, s, d, got[dst], w);
          }
  };
  {  // test_gpu_rotary_f32_small_split_half: [1,2,4,8], [X, cos, sin] -> position 0
    const int B = 1, H = 2, S = 4, D = 8, rows = 16;
    std::vector<float> x(B * H * S * D);
    for (size_t i = 0; i < x.size(); ++i) x[i] = (float)i * 0.0125f - 0.25f;
    std::vector<float> c, sn;
    rope_tables(rows, D, 1e4, c, sn);
    DeviceTensor xd = f32_tensor(x, shp({B, H, S, D}));
    DeviceTensor cd = f32_tensor(c, shp({rows, D / 2})), sd = f32_tensor(sn, shp({rows, D / 2}));
    auto out = must(dispatch_rotary_embedding(rt, {&xd, &cd, &sd}, {}, nullptr), "small split-half");
    REQUIRE(out.size() == 1 && out[0].shape == xd.shape && out[0].dtype == DataType::Float, "output");
    check(x, B, H, S, D, false, c, sn, rows, 0, false, host_f32(out[0]), "small split-half");
  }
  {  // test_gpu_rotary_f32_decode_step_interleaved: [2,4,1,16] at 37 from position_ids
    const int B = 2, H = 4, S = 1, D = 16, rows = 64;
    std::vector<float> x(B * H * S * D);
    for (size_t i = 0; i < x.size(); ++i) x[i] = std::sin((float)i * 0.07f);
    std::vector<float> c, sn;
    rope_tables(rows, D, 1e4, c, sn);
    DeviceTensor xd = f32_tensor(x, shp({B, H, S, D}));
    DeviceTensor cd = f32_tensor(c, shp({rows, D / 2})), sd = f32_tensor(sn, shp({rows, D / 2}));
    DeviceTensor pos = i64_tensor({37}, shp({1, 1}));
    auto out = must(dispatch_rotary_embedding(rt, {&xd, &pos, &cd, &sd},
                                              {AttributeProto::make_int("interleaved", 1)}, nullptr),
                    "decode interleaved");
    check(x, B, H, S, D, false, c, sn, rows, 37, true, host_f32(out[0]), "decode interleaved");
  }
  {  // test_gpu_rotary_bf16_gemma_shape: [1,8,8,128] bf16 against the f32 op within 1e-2
    const int B = 1, H = 8, S = 8, D = 128, rows = 32;
    std::vector<float> x(B * H * S * D);
    for (size_t i = 0; i < x.size(); ++i) x[i] = std::cos((float)i * 0.001f) * 0.5f;
    DeviceTensor xd = bf16_tensor(x, shp({B, H, S, D}));  // x now holds the bf16 values
    std::vector<float> c, sn;
    rope_tables(rows, D, 1e4, c, sn);
    DeviceTensor cd = f32_tensor(c, shp({rows, D / 2})), sd = f32_tensor(sn, shp({rows, D / 2}));
    auto out = must(dispatch_rotary_embedding(rt, {&xd, &cd, &sd}, {}, nullptr), "bf16 gemma");
    REQUIRE(out[0].dtype == DataType::BFloat16, "bf16 output");
    auto raw = must(out[0].to_host(), "bf16 read");
    std::vector<float> want = x;
    std::vector<int64_t> ids(S);
    for (int s = 0; s < S; ++s) ids[s] = s;
    REQUIRE(sai_or_apply_rope(want.data(), B, H, S, D, c.data(), sn.data(), rows, D / 2, ids.data(), S, 0, D) == 0, "oracle");
    for (size_t i = 0; i < want.size(); ++i) {
      uint16_t b;
      std::memcpy(&b, raw.data() + 2 * i, 2);
      REQUIRE(std::fabs(sai_or_bf16_to_f32(b) - want[i]) < 1e-2f, "bf16 element %zu", i);
      REQUIRE(b == sai_or_f32_to_bf16(want[i]), "bf16 element %zu not the rounded oracle value", i);
    }
  }
  {  // rank 3 [B, S, H*D]: rows (b, s, h), num_heads from the attribute or the tables
    const int B = 2, H = 3, S = 5, D = 64, rows = 40;
    std::vector<float> x = gauss(g, (size_t)B * S * H * D);
    std::vector<float> c, sn;
    rope_tables(rows, D, 5e5, c, sn);
    DeviceTensor xd = f32_tensor(x, shp({B, S, H * D}));
    DeviceTensor cd = f32_tensor(c, shp({rows, D / 2})), sd = f32_tensor(sn, shp({rows, D / 2}));
    DeviceTensor pos = i64_tensor({11, 99, 3}, shp({3}));  // only the first id counts
    auto a = must(dispatch_rotary_embedding(rt, {&xd, &pos, &cd, &sd}, {AttributeProto::make_int("num_heads", H)}, nullptr), "rank3 attr");
    check(x, B, H, S, D, true, c, sn, rows, 11, false, host_f32(a[0]), "rank3 attr");
    auto b = must(dispatch_rotary_embedding(rt, {&xd, &pos, &cd, &sd}, {}, nullptr), "rank3 derived");
    check(x, B, H, S, D, true, c, sn, rows, 11, false, host_f32(b[0]), "rank3 derived");
    // bf16 tables are read as their f32 values (the reference casts them)
    std::vector<float> cb = c, sb = sn;
    DeviceTensor cbd = bf16_tensor(cb, shp({rows, D / 2})), sbd = bf16_tensor(sb, shp({rows, D / 2}));
    auto t = must(dispatch_rotary_embedding(rt, {&xd, &pos, &cbd, &sbd}, {}, nullptr), "bf16 tables");
    check(x, B, H, S, D, true, cb, sb, rows, 11, false, host_f32(t[0]), "bf16 tables");
  }
  {  // no position_ids: the cache's current position
    const int D = 128, rows = 64;
    auto cache = must(GpuKvCache::allocate(rt, 1, 1, D, rows, KvQuant::Int8, {LayerKind::global()}, 1), "cache");
    std::vector<float> k1 = gauss(g, 7 * D), v1 = gauss(g, 7 * D);
    DeviceTensor kd = f32_tensor(k1, shp({1, 7, D})), vd = f32_tensor(v1, shp({1, 7, D}));
    must(cache.append(0, kd, vd), "append 7");
    must(cache.advance_position(), "advance");
    KvCacheDispatchCtx ctx{&cache, 0};
    std::vector<float> x = gauss(g, 4 * 2 * D);
    std::vector<float> c, sn;
    rope_tables(rows, D, 1e4, c, sn);
    DeviceTensor xd = f32_tensor(x, shp({1, 4, 2, D}));
    DeviceTensor cd = f32_tensor(c, shp({rows, D / 2})), sd = f32_tensor(sn, shp({rows, D / 2}));
    auto out = must(dispatch_rotary_embedding(rt, {&xd, &cd, &sd}, {}, &ctx), "cache position");
    check(x, 1, 4, 2, D, false, c, sn, rows, 7, false, host_f32(out[0]), "cache position");
  }
  {  // errors (rotary.rs:150-256, gpu_executor.rs:724-745)
    std::vector<float> c, sn;
    rope_tables(4, 8, 1e4, c, sn);
    DeviceTensor cd = f32_tensor(c, shp({4, 4})), sd = f32_tensor(sn, shp({4, 4}));
    DeviceTensor x7 = f32_tensor(std::vector<float>(7), shp({1, 1, 1, 7}));
    DeviceTensor c3 = f32_tensor(std::vector<float>(3), shp({1, 3}));
    struct E {
      std::vector<const DeviceTensor*> in;
      std::vector<AttributeProto> attrs;
      const char* msg;
    };
    DeviceTensor x8 = f32_tensor(std::vector<float>(8 * 5), shp({1, 1, 5, 8}));
    DeviceTensor x2 = f32_tensor(std::vector<float>(8), shp({1, 8}));
    DeviceTensor x3 = f32_tensor(std::vector<float>(2 * 12), shp({1, 2, 12}));
    DeviceTensor xi = i64_tensor({0, 0, 0, 0}, shp({1, 1, 1, 4}));
    DeviceTensor ci = i64_tensor(std::vector<int64_t>(16), shp({4, 4}));
    const std::vector<E> cases = {
        {{&x7, &c3, &c3}, {}, "internal error: ROCm RotaryEmbedding: HIP rotary_gpu: head_dim must be a positive even integer failed: code -1"},
        {{&x8, &cd, &sd}, {}, "internal error: ROCm RotaryEmbedding: HIP rotary_gpu: position + seq_len exceeds cos/sin table length failed: code -1"},
        {{&x2, &cd, &sd}, {}, "internal error: ROCm RotaryEmbedding: HIP rotary_gpu: x must be rank-3 or rank-4 failed: code -1"},
        {{&x3, &cd, &sd}, {}, "internal error: ROCm RotaryEmbedding: HIP rotary_gpu: rank-3 input requires num_heads_for_rank3 failed: code -1"},
        {{&x3, &cd, &sd}, {AttributeProto::make_int("num_heads", 0)}, "internal error: ROCm RotaryEmbedding: HIP rotary_gpu: num_heads must be > 0 for rank-3 input failed: code -1"},
        {{&x3, &cd, &sd}, {AttributeProto::make_int("num_heads", 5)}, "internal error: ROCm RotaryEmbedding: HIP rotary_gpu: hidden not divisible by num_heads (rank-3) failed: code -1"},
        {{&xi, &cd, &sd}, {}, "internal error: ROCm RotaryEmbedding: HIP rotary_gpu: unsupported dtype (need Float or BFloat16) failed: code -1"},
        {{&x8, &ci, &ci}, {}, "internal error: ROCm RotaryEmbedding: HIP rotary_gpu: cos/sin tables must be Float failed: code -1"},
        {{&x8, &c3, &c3}, {}, "internal error: ROCm RotaryEmbedding: HIP rotary_gpu: cos/sin inner dim must equal head_dim / 2 failed: code -1"},
        {{&x8}, {}, "internal error: GPU RotaryEmbedding: missing input 'cos_cache'"},
        {{nullptr, &cd, &sd}, {}, "internal error: GPU RotaryEmbedding: missing input 'X'"},
        {{&x8, nullptr, &cd, &sd}, {}, "internal error: GPU RotaryEmbedding: missing input 'position_ids'"},
    };
    for (const E& e : cases) {
      OpError err = must_fail(dispatch_rotary_embedding(rt, e.in, e.attrs, nullptr), e.msg);
      REQUIRE(err.to_string() == e.msg, "got '%s'", err.to_string().c_str());
    }
  }
}

// precompute_rope_tables (model_loader/gemma.rs:458-472) against the oracle.
void gpu_rope_tables() {
  RocmRuntime& rt = runtime();
  for (auto [max_pos, half, theta] : {std::tuple<int, int, float>{16, 4, 1e4f}, {4096, 64, 1e6f}, {300, 128, 5e5f}}) {
    auto t = must(precompute_rope_tables(rt, (size_t)max_pos, (size_t)half, theta), "tables");
    REQUIRE(t.first.shape == shp({max_pos, half}) && t.first.dtype == DataType::BFloat16, "shape/dtype");
    std::vector<uint16_t> wc((size_t)max_pos * half), ws(wc.size());
    sai_or_rope_tables_bf16(max_pos, half, theta, wc.data(), ws.data());
    auto gc = must(t.first.to_host(), "cos"), gs = must(t.second.to_host(), "sin");
    REQUIRE(gc.size() == wc.size() * 2 && std::memcmp(gc.data(), wc.data(), gc.size()) == 0,
            "cos table %dx%d differs from the oracle", max_pos, half);
    REQUIRE(std::memcmp(gs.data(), ws.data(), gs.size()) == 0, "sin table %dx%d differs", max_pos, half);
  }
}

// appends into a logical cache and attends over its dequantised contents.
// lw > 0: layer 1 is a sliding-window layer of lw keys; mw: the nodes'
// local_window_size (-1: none).
static void session(KvQuant quant, bool bf16, int B, int Hq, int Hkv, int D, int prefill,
                    int steps, unsigned seed, int lw = 0, int mw = -1) {
  RocmRuntime& rt = runtime();
  const int layers = 2, rows = 512, t_cap = prefill + steps;
  std::vector<float> cs, sn;
  rope_tables(rows, D, 10000.0, cs, sn);
  DeviceTensor dcos = f32_tensor(cs, shp({rows, D / 2})), dsin = f32_tensor(sn, shp({rows, D / 2}));
  std::vector<LayerKind> kinds(layers, LayerKind::global());
  if (lw > 0) kinds[1] = LayerKind::sliding_window((size_t)lw);
  GpuKvCache cache = must(GpuKvCache::allocate(rt, layers, Hkv, D, t_cap, quant, kinds, B),
                          "allocate");
  const int q8 = quant == KvQuant::Int8 ? 1 : 2;
  const size_t rowsz = (size_t)B * Hkv * t_cap;
  struct Logical {
    std::vector<int8_t> k8, v8;
    std::vector<uint8_t> k4, v4;
    std::vector<float> ks, vs;
    std::vector<uint16_t> ksz, vsz;
  };
  std::vector<Logical> lc(layers);
  for (Logical& l : lc) {
    l.k8.resize(rowsz * D);
    l.v8.resize(rowsz * D);
    l.k4.resize(rowsz * D / 2);
    l.v4.resize(rowsz * D / 2);
    l.ks.resize(rowsz);
    l.vs.resize(rowsz);
    l.ksz.resize(rowsz * D / 16);
    l.vsz.resize(rowsz * D / 16);
  }
  std::vector<AttributeProto> attrs = {AttributeProto::make_int("num_heads", Hq),
                                       AttributeProto::make_int("kv_num_heads", Hkv)};
  if (mw != -1) attrs.push_back(AttributeProto::make_int("local_window_size", mw));
  std::mt19937_64 gen(seed);
  int pos = 0;
  const int passes = (prefill > 0 ? 1 : 0) + steps;
  for (int pass = 0; pass < passes; ++pass) {
    const int S = (prefill > 0 && pass == 0) ? prefill : 1;
    KvCacheDispatchCtx ctx{&cache, 0};
    for (int layer = 0; layer < layers; ++layer) {
      std::vector<float> q = gauss(gen, (size_t)B * S * Hq * D);
      std::vector<float> k = gauss(gen, (size_t)B * S * Hkv * D);
      std::vector<float> v = gauss(gen, (size_t)B * S * Hkv * D);
      const auto sq = shp({B, S, (int64_t)Hq * D}), skv = shp({B, S, (int64_t)Hkv * D});
      DeviceTensor dq = bf16 ? bf16_tensor(q, sq) : f32_tensor(q, sq);
      DeviceTensor dk = bf16 ? bf16_tensor(k, skv) : f32_tensor(k, skv);
      DeviceTensor dv = bf16 ? bf16_tensor(v, skv) : f32_tensor(v, skv);
      auto outs = must(dispatch_gqa(rt, {&dq, &dk, &dv, nullptr, nullptr, nullptr, nullptr, &dcos, &dsin},
                                    attrs, &ctx),
                       "dispatch_gqa");
      REQUIRE(ctx.next_layer_idx == (size_t)layer + 1, "layer counter");
      // attn_out in Q's dtype (gpu_gqa: dt = q.dtype, attention.rs:835)
      REQUIRE(outs[0].dtype == (bf16 ? DataType::BFloat16 : DataType::Float), "attn_out dtype");
      std::vector<float> got = host_values(outs[0]);
      // oracle
      Logical& l = lc[layer];
      std::vector<int32_t> start(B, pos), lens(B, pos + S);
      REQUIRE(sai_or_kv_append(k.data(), v.data(), B, S, Hkv, D, start.data(), cs.data(), sn.data(),
                               rows, 1, 0, q8, t_cap, q8 == 1 ? (void*)l.k8.data() : l.k4.data(),
                               q8 == 1 ? (void*)l.v8.data() : l.v4.data(), l.ks.data(), l.vs.data(),
                               l.ksz.data(), l.vsz.data()) == 0,
              "oracle append");
      std::vector<float> kd(rowsz * D), vd(rowsz * D);
      REQUIRE(sai_or_kv_dequant(B, Hkv, D, q8, t_cap, lens.data(),
                                q8 == 1 ? (const void*)l.k8.data() : l.k4.data(),
                                q8 == 1 ? (const void*)l.v8.data() : l.v4.data(), l.ks.data(),
                                l.vs.data(), l.ksz.data(), l.vsz.data(), kd.data(), vd.data()) == 0,
              "oracle dequant");
      std::vector<float> want((size_t)B * S * Hq * D);
      REQUIRE(sai_or_gqa_cached_window(q.data(), B, S, Hq, Hkv, D, lens.data(), t_cap, kd.data(),
                                       vd.data(), cs.data(), sn.data(), rows, 1, 0, 0, 0.0f,
                                       layer == 1 ? lw : 0, mw, want.data()) == 0,
              "oracle gqa");
      char what[96];
      std::snprintf(what, sizeof what, "pass %d layer %d output", pass, layer);
      if (bf16)
        close_bf16(got, want, what);
      else
        close(got, want, what);
      // the cache holds exactly the oracle's codes: dequantised values agree bit for bit
      for (int b = 0; b < B; ++b)
        for (int h = 0; h < Hkv; ++h) {
          auto kv = must(cache.read_dequantized(layer, b, h, 0, pos + S), "read");
          const size_t base = ((size_t)b * Hkv + h) * t_cap * D;
          REQUIRE(std::memcmp(kv.first.data(), kd.data() + base, (size_t)(pos + S) * D * 4) == 0,
                  "pass %d layer %d K cache (b %d h %d) differs from the oracle", pass, layer, b, h);
          REQUIRE(std::memcmp(kv.second.data(), vd.data() + base, (size_t)(pos + S) * D * 4) == 0,
                  "pass %d layer %d V cache (b %d h %d) differs from the oracle", pass, layer, b, h);
        }
    }
    must(cache.advance_position(), "advance");
    pos += S;
    REQUIRE(cache.current_position() == (size_t)pos, "position %zu != %d", cache.current_position(), pos);
  }
}

static void gpu_session_int8_prefill_decode() { session(KvQuant::Int8, false, 2, 8, 2, 128, 40, 6, 11); }
static void gpu_session_int8_bf16_d64() { session(KvQuant::Int8, true, 3, 8, 2, 64, 17, 4, 12); }
static void gpu_session_int4_decode() { session(KvQuant::Int4, false, 2, 16, 2, 128, 0, 24, 13); }
static void gpu_session_int4_prefill_decode() { session(KvQuant::Int4, true, 2, 8, 2, 128, 37, 5, 15); }
static void gpu_session_int4_bf16_group4() { session(KvQuant::Int4, true, 1, 8, 2, 128, 0, 20, 14); }
static void gpu_session_int8_windows() { session(KvQuant::Int8, false, 2, 8, 2, 128, 150, 6, 16, 30, 40); }
static void gpu_session_int4_layer_window() { session(KvQuant::Int4, true, 2, 8, 2, 128, 100, 5, 17, 33); }

// The CPU ops' contract with explicit past K/V (op_group_query_attention,
// ops/microsoft.rs:1082-1190; op_multi_head_attention, :806-925): present
// K/V bit-exact against the oracle's restatement of the op (sai_or_gqa); the
// attention within the parity bar of the oracle over the dequantised int8
// cache that holds the same past and new rows.
static void cpu_op_case(bool mha, int B, int Hq, int Hkv, int D, int S, int P, bool rot, bool il,
                        bool has_scale, unsigned seed) {
  RocmRuntime& rt = runtime();
  std::mt19937_64 gen(seed);
  const int rows = P + S + 5;
  std::vector<float> cs, sn;
  rope_tables(rows, D, 10000.0, cs, sn);
  std::vector<float> q = gauss(gen, (size_t)B * S * Hq * D);
  std::vector<float> k = gauss(gen, (size_t)B * S * Hkv * D);
  std::vector<float> v = gauss(gen, (size_t)B * S * Hkv * D);
  std::vector<float> pk = gauss(gen, (size_t)B * Hkv * P * D);
  std::vector<float> pv = gauss(gen, (size_t)B * Hkv * P * D);
  DeviceTensor dq = f32_tensor(q, shp({B, S, (int64_t)Hq * D}));
  DeviceTensor dk = f32_tensor(k, shp({B, S, (int64_t)Hkv * D}));
  DeviceTensor dv = f32_tensor(v, shp({B, S, (int64_t)Hkv * D}));
  DeviceTensor dpk = f32_tensor(pk, shp({B, Hkv, P, D})), dpv = f32_tensor(pv, shp({B, Hkv, P, D}));
  DeviceTensor dcos = f32_tensor(cs, shp({rows, D / 2})), dsin = f32_tensor(sn, shp({rows, D / 2}));
  const std::optional<float> scale = has_scale ? std::optional<float>(0.07f) : std::nullopt;
  const DeviceTensor* past_k = P > 0 ? &dpk : nullptr;
  const DeviceTensor* past_v = P > 0 ? &dpv : nullptr;
  AttentionOutputs o =
      mha ? must(op_multi_head_attention(rt, {&dq, &dk, &dv, nullptr, nullptr, nullptr, past_k, past_v},
                                         Hq, scale),
                 "op_multi_head_attention")
          : must(op_group_query_attention(rt, {&dq, &dk, &dv, past_k, past_v, nullptr, nullptr,
                                               rot ? &dcos : nullptr, rot ? &dsin : nullptr},
                                          Hq, Hkv, scale, -1, rot, il),
                 "op_group_query_attention");
  REQUIRE(o.attn.shape == shp({B, S, (int64_t)Hq * D}), "attn shape");
  REQUIRE(o.present_key.shape == shp({B, Hkv, P + S, D}), "present shape");
  // present: exact
  const int T = P + S;
  std::vector<float> w_attn((size_t)B * S * Hq * D), w_pk((size_t)B * Hkv * T * D), w_pv(w_pk.size());
  REQUIRE(sai_or_gqa(q.data(), k.data(), v.data(), B, S, Hq * D, Hkv * D, P ? pk.data() : nullptr,
                     P ? pv.data() : nullptr, P, cs.data(), sn.data(), rows, D / 2, Hq, Hkv,
                     has_scale ? 1 : 0, 0.07f, -1, rot ? 1 : 0, il ? 1 : 0, w_attn.data(), w_pk.data(),
                     w_pv.data()) == 0,
          "oracle op");
  const std::vector<float> g_pk = host_f32(o.present_key), g_pv = host_f32(o.present_value);
  REQUIRE(std::memcmp(g_pk.data(), w_pk.data(), w_pk.size() * 4) == 0, "present_key differs from the oracle");
  REQUIRE(std::memcmp(g_pv.data(), w_pv.data(), w_pv.size() * 4) == 0, "present_value differs from the oracle");
  // attention: the oracle over the int8 cache of the same rows
  std::vector<int8_t> k8((size_t)B * Hkv * T * D), v8(k8.size());
  std::vector<float> ks((size_t)B * Hkv * T), vs(ks.size());
  std::vector<int32_t> zero(B, 0), at_p(B, P), lens(B, T);
  if (P > 0) {
    std::vector<float> rk((size_t)B * P * Hkv * D), rv(rk.size());  // past as rows
    for (int b = 0; b < B; ++b)
      for (int h = 0; h < Hkv; ++h)
        for (int t = 0; t < P; ++t)
          for (int d = 0; d < D; ++d) {
            const size_t src = (((size_t)b * Hkv + h) * P + t) * D + d;
            const size_t dst = (((size_t)b * P + t) * Hkv + h) * D + d;
            rk[dst] = pk[src];
            rv[dst] = pv[src];
          }
    REQUIRE(sai_or_kv_append(rk.data(), rv.data(), B, P, Hkv, D, zero.data(), nullptr, nullptr, 0, 0, 0,
                             1, T, k8.data(), v8.data(), ks.data(), vs.data(), nullptr, nullptr) == 0,
            "oracle past append");
  }
  REQUIRE(sai_or_kv_append(k.data(), v.data(), B, S, Hkv, D, at_p.data(), cs.data(), sn.data(), rows,
                           rot ? 1 : 0, il ? 1 : 0, 1, T, k8.data(), v8.data(), ks.data(), vs.data(),
                           nullptr, nullptr) == 0,
          "oracle new append");
  std::vector<float> kd((size_t)B * Hkv * T * D), vd(kd.size());
  REQUIRE(sai_or_kv_dequant(B, Hkv, D, 1, T, lens.data(), k8.data(), v8.data(), ks.data(), vs.data(),
                            nullptr, nullptr, kd.data(), vd.data()) == 0,
          "oracle dequant");
  std::vector<float> want((size_t)B * S * Hq * D);
  REQUIRE(sai_or_gqa_cached(q.data(), B, S, Hq, Hkv, D, lens.data(), T, kd.data(), vd.data(), cs.data(),
                            sn.data(), rows, rot ? 1 : 0, il ? 1 : 0, has_scale ? 1 : 0, 0.07f,
                            want.data()) == 0,
          "oracle attention");
  close(host_f32(o.attn), want, mha ? "MHA attention" : "GQA attention");
}

void gpu_cpu_op_gqa_with_past() {
  cpu_op_case(false, 2, 8, 2, 128, 1, 37, true, false, false, 41);   // decode step
  cpu_op_case(false, 1, 4, 4, 64, 5, 0, true, true, false, 42);      // first chunk, no past
  cpu_op_case(false, 2, 8, 1, 128, 3, 20, false, false, true, 43);   // no RoPE, explicit scale
  cpu_op_case(false, 1, 16, 2, 128, 70, 130, true, false, false, 44);  // prefill chunk over a past
}

void gpu_cpu_op_mha_with_past() {
  cpu_op_case(true, 2, 4, 4, 64, 3, 0, false, false, false, 51);
  cpu_op_case(true, 1, 2, 2, 128, 1, 17, false, false, true, 52);
  cpu_op_case(true, 2, 8, 8, 64, 40, 25, false, false, false, 53);
}

// The reference's op tests (ops/microsoft.rs:1541-1600, :1602-1830, :2000-2060)
// restated at head_dim 64: shapes of present across calls, Q = 0 giving the
// mean of the visible values, and the error contract.
void gpu_cpu_op_kats() {
  RocmRuntime& rt = runtime();
  const int D = 64;
  {  // mha_basic_two_heads_no_cache: Q = 0 -> q0 = v0, q1 = (v0 + v1) / 2
    std::vector<float> q(2 * 2 * D, 0.0f), k, v;
    std::mt19937_64 gen(7);
    k = gauss(gen, 2 * 2 * D);
    v = gauss(gen, 2 * 2 * D);
    DeviceTensor dq = f32_tensor(q, shp({1, 2, 2 * D})), dk = f32_tensor(k, shp({1, 2, 2 * D})),
                 dv = f32_tensor(v, shp({1, 2, 2 * D}));
    AttentionOutputs o = must(op_multi_head_attention(rt, {&dq, &dk, &dv}, 2, std::nullopt), "mha");
    REQUIRE(o.attn.shape == shp({1, 2, 2 * D}) && o.present_key.shape == shp({1, 2, 2, D}) &&
                o.present_value.shape == shp({1, 2, 2, D}),
            "shapes");
    const std::vector<float> a = host_f32(o.attn);
    for (int h = 0; h < 2; ++h)
      for (int d = 0; d < D; ++d) {
        const float v0 = v[(size_t)h * D + d], v1 = v[(size_t)(2 + h) * D + d];
        REQUIRE(std::fabs(a[(size_t)h * D + d] - v0) < 0.02f, "q0 = v0 (h %d d %d)", h, d);
        REQUIRE(std::fabs(a[(size_t)(2 + h) * D + d] - 0.5f * (v0 + v1)) < 0.02f, "q1 = mean (h %d d %d)", h, d);
      }
  }
  {  // gqa_kv_cache_mutation_across_calls: present grows 2 -> 3
    DeviceTensor q1 = f32_tensor(std::vector<float>(2 * 4 * D, 0.0f), shp({1, 2, 4 * D}));
    DeviceTensor k1 = f32_tensor(std::vector<float>(2 * 2 * D, 1.0f), shp({1, 2, 2 * D}));
    DeviceTensor v1 = f32_tensor(std::vector<float>(2 * 2 * D, 2.0f), shp({1, 2, 2 * D}));
    AttentionOutputs o1 = must(op_group_query_attention(rt, {&q1, &k1, &v1}, 4, 2, std::nullopt, -1, false, false),
                               "call 1");
    REQUIRE(o1.present_key.shape == shp({1, 2, 2, D}), "present 1");
    DeviceTensor q2 = f32_tensor(std::vector<float>(4 * D, 0.0f), shp({1, 1, 4 * D}));
    DeviceTensor k2 = f32_tensor(std::vector<float>(2 * D, 3.0f), shp({1, 1, 2 * D}));
    DeviceTensor v2 = f32_tensor(std::vector<float>(2 * D, 4.0f), shp({1, 1, 2 * D}));
    AttentionOutputs o2 = must(op_group_query_attention(rt, {&q2, &k2, &v2, &o1.present_key, &o1.present_value},
                                                        4, 2, std::nullopt, -1, false, false),
                               "call 2");
    REQUIRE(o2.present_key.shape == shp({1, 2, 3, D}), "present 2");
    // Q = 0: uniform over the 3 keys -> (2 + 2 + 4) / 3 in every value dim
    for (float x : host_f32(o2.attn)) REQUIRE(std::fabs(x - 8.0f / 3.0f) < 0.02f, "mean %g", x);
  }
  {  // errors
    DeviceTensor q = f32_tensor(std::vector<float>(4 * D, 0.0f), shp({1, 1, 4 * D}));
    DeviceTensor k = f32_tensor(std::vector<float>(2 * D, 0.0f), shp({1, 1, 2 * D}));
    DeviceTensor bad_past = f32_tensor(std::vector<float>(2 * 2 * D, 0.0f), shp({1, 2, 2 * D}));
    DeviceTensor past = f32_tensor(std::vector<float>(2 * D, 0.0f), shp({1, 2, 1, D}));
    auto gqa = [&](std::vector<const DeviceTensor*> in, int64_t lw, bool rot) {
      return op_group_query_attention(rt, in, 4, 2, std::nullopt, lw, rot, false);
    };
    OpError e = must_fail(gqa({&q, &k, &k}, 512, false), "local window");
    REQUIRE(e.kind == OpError::Kind::InvalidAttribute &&
                e.message == "GroupQueryAttention: local_window_size != -1 not supported in this tier", "%s", e.to_string().c_str());
    e = must_fail(gqa({&q, &k}, -1, false), "missing value");
    REQUIRE(e.message == "GroupQueryAttention: missing value", "%s", e.to_string().c_str());
    e = must_fail(gqa({&q, &k, &k}, -1, true), "do_rotary without tables");
    REQUIRE(e.message == "GroupQueryAttention: do_rotary=1 but cos_cache is missing", "%s", e.to_string().c_str());
    e = must_fail(gqa({&q, &k, &k, &bad_past}, -1, false), "past rank");
    REQUIRE(e.message == "GroupQueryAttention: past_key must be rank-4", "%s", e.to_string().c_str());
    e = must_fail(gqa({&q, &k, &k, &past}, -1, false), "past_value missing");
    REQUIRE(e.message == "GroupQueryAttention: past_key / past_value sequence mismatch", "%s", e.to_string().c_str());
    DeviceTensor odd = f32_tensor(std::vector<float>(3 * D, 0.0f), shp({1, 1, 3 * D}));
    e = must_fail(op_group_query_attention(rt, {&odd, &k, &k}, 3, 2, std::nullopt, -1, false, false), "heads");
    REQUIRE(e.kind == OpError::Kind::InvalidAttribute, "%s", e.to_string().c_str());
    DeviceTensor m = f32_tensor(std::vector<float>(4 * D, 0.0f), shp({1, 1, 4 * D}));
    DeviceTensor r2 = f32_tensor(std::vector<float>(4 * D, 0.0f), shp({1, 4 * D}));
    e = must_fail(op_multi_head_attention(rt, {&r2, &m, &m}, 2, std::nullopt), "mha rank");
    REQUIRE(e.message == "MultiHeadAttention: Q/K/V must be rank-3 (B, Sq, hidden)", "%s", e.to_string().c_str());
    e = must_fail(op_multi_head_attention(rt, {&m, &m, &m}, 3, std::nullopt), "mha heads");
    REQUIRE(e.message == "MultiHeadAttention: hidden not divisible by num_heads", "%s", e.to_string().c_str());
    DeviceTensor mp = f32_tensor(std::vector<float>(4 * D, 0.0f), shp({1, 4, 1, D}));
    e = must_fail(op_multi_head_attention(rt, {&m, &m, &m, nullptr, nullptr, nullptr, &mp}, 4, std::nullopt),
                  "mha missing past_value");
    REQUIRE(e.message == "MultiHeadAttention: past_key/past_value sequence length mismatch", "%s", e.to_string().c_str());
    DeviceTensor d3 = f32_tensor(std::vector<float>(4 * 24, 0.0f), shp({1, 1, 4 * 24}));
    e = must_fail(op_multi_head_attention(rt, {&d3, &d3, &d3}, 4, std::nullopt), "mha head_dim 24");
    REQUIRE(e.kind == OpError::Kind::UnsupportedOp, "%s", e.to_string().c_str());
  }
}

// RoPE of [B, S, H*D] rows at positions start + s, through the oracle's
// apply_rope on the [B, H, S, D] view.
static void oracle_rope_bshd(std::vector<float>& x, int B, int S, int H, int D, int start,
                             const std::vector<float>& cs, const std::vector<float>& sn, int rows) {
  std::vector<float> v(x.size());
  for (int b = 0; b < B; ++b)
    for (int s = 0; s < S; ++s)
      for (int h = 0; h < H; ++h)
        for (int d = 0; d < D; ++d)
          v[(((size_t)b * H + h) * S + s) * D + d] = x[(((size_t)b * S + s) * H + h) * D + d];
  std::vector<int64_t> ids(S);
  for (int s = 0; s < S; ++s) ids[s] = start + s;
  REQUIRE(sai_or_apply_rope(v.data(), B, H, S, D, cs.data(), sn.data(), rows, D / 2, ids.data(), S, 0, D) == 0,
          "oracle rope");
  for (int b = 0; b < B; ++b)
    for (int s = 0; s < S; ++s)
      for (int h = 0; h < H; ++h)
        for (int d = 0; d < D; ++d)
          x[(((size_t)b * S + s) * H + h) * D + d] = v[(((size_t)b * H + h) * S + s) * D + d];
}

// session.rs:579-593
void cpu_layer_kinds_for_gemma() {
  const auto k = layer_kinds_for_gemma(6, 16, 2);
  REQUIRE(k.size() == 6, "count");
  for (size_t i = 0; i < 6; ++i) {
    const bool global = (i + 1) % 2 == 0;
    REQUIRE((k[i].tag == LayerKind::Tag::Global) == global, "layer %zu", i);
    if (!global) REQUIRE(k[i].window == 16, "window");
  }
  const auto k5 = layer_kinds_for_gemma(5, 0, 6);  // last layer global, window at least 1
  REQUIRE(k5[4].tag == LayerKind::Tag::Global && k5[0].window == 1, "pattern 6 of 5 layers");
  REQUIRE(SessionError::execution("x").to_string() == "execution failed: x", "display");
}

// A Gemma-shaped attention graph driven through GpuSession: per layer two
// RotaryEmbedding nodes ([x, cos, sin]: the start is the cache position) and
// one GroupQueryAttention node (local_window_size on the sliding layers);
// layer kinds from layer_kinds_for_gemma. A prefill pass, decode passes, then
// reset_kv_cache and a fresh pass, each checked against the oracle (RoPE by
// apply_rope, the int8 cache by kv_append without rotation, attention with
// both window rules).
// A Gemma-shaped graph (per layer: RoPE on q and k, then GQA; sliding layers
// every other one) through GpuSession: prefill and decode passes against the
// oracle, reset, then the executor's error paths.
void gemma_graph_session(int Hq, int Hkv, int D, double theta, uint64_t seed) {
  const int L = 4, B = 2, W = 24, rows = 160;
  SessionConfig cfg;
  cfg.num_hidden_layers = L;
  cfg.num_key_value_heads = Hkv;
  cfg.head_dim = D;
  cfg.max_seq_len = 128;
  cfg.max_batch = B;
  cfg.sliding_window = W;
  cfg.sliding_window_pattern = 2;
  std::vector<ExecutionNode> graph;
  std::vector<std::string> outs;
  for (int l = 0; l < L; ++l) {
    const std::string i = std::to_string(l);
    graph.push_back({"rope_q" + i, "RotaryEmbedding", {"q" + i, "cos", "sin"}, {"qr" + i},
                     {AttributeProto::make_int("rotary_embedding_dim", D), AttributeProto::make_int("interleaved", 0)}});
    graph.push_back({"rope_k" + i, "RotaryEmbedding", {"k" + i, "cos", "sin"}, {"kr" + i},
                     {AttributeProto::make_int("rotary_embedding_dim", D), AttributeProto::make_int("interleaved", 0)}});
    std::vector<AttributeProto> a = {AttributeProto::make_int("num_heads", Hq), AttributeProto::make_int("kv_num_heads", Hkv)};
    if (l % 2 == 0) a.push_back(AttributeProto::make_int("local_window_size", W));
    graph.push_back({"gqa" + i, "GroupQueryAttention", {"qr" + i, "kr" + i, "v" + i, "", ""},
                     {"attn" + i, "present_k" + i, "present_v" + i}, a});
    outs.push_back("attn" + i);
  }
  auto session = must(GpuSession::create(0, cfg, graph, outs), "GpuSession::create");
  REQUIRE(session->layer_kinds()[0].tag == LayerKind::Tag::SlidingWindow && session->layer_kinds()[1].tag == LayerKind::Tag::Global,
          "layer kinds");
  std::vector<float> cs, sn;
  rope_tables(rows, D, theta, cs, sn);
  // oracle state per layer: int8 codes of the rotated keys
  const int T = 128;
  struct Lay { std::vector<int8_t> k8, v8; std::vector<float> ks, vs; };
  std::vector<Lay> lay(L);
  auto clear = [&]() {
    for (Lay& x : lay) {
      x.k8.assign((size_t)B * Hkv * T * D, 0); x.v8.assign(x.k8.size(), 0);
      x.ks.assign((size_t)B * Hkv * T, 0.0f); x.vs.assign(x.ks.size(), 0.0f);
    }
  };
  clear();
  std::mt19937_64 gen(seed);
  int pos = 0;
  auto pass = [&](int S, const char* what) {
    std::vector<std::pair<std::string, DeviceTensor>> in;
    in.emplace_back("cos", f32_tensor(cs, shp({rows, D / 2})));
    in.emplace_back("sin", f32_tensor(sn, shp({rows, D / 2})));
    std::vector<std::vector<float>> qs(L), ks(L), vs(L);
    for (int l = 0; l < L; ++l) {
      const std::string i = std::to_string(l);
      qs[l] = gauss(gen, (size_t)B * S * Hq * D);
      ks[l] = gauss(gen, (size_t)B * S * Hkv * D);
      vs[l] = gauss(gen, (size_t)B * S * Hkv * D);
      in.emplace_back("q" + i, f32_tensor(qs[l], shp({B, S, (int64_t)Hq * D})));
      in.emplace_back("k" + i, f32_tensor(ks[l], shp({B, S, (int64_t)Hkv * D})));
      in.emplace_back("v" + i, f32_tensor(vs[l], shp({B, S, (int64_t)Hkv * D})));
    }
    auto got = must(session->run(std::move(in)), what);
    REQUIRE(got.size() == (size_t)L, "%s: outputs", what);
    for (int l = 0; l < L; ++l) {
      std::vector<float> q = qs[l], k = ks[l];
      oracle_rope_bshd(q, B, S, Hq, D, pos, cs, sn, rows);
      oracle_rope_bshd(k, B, S, Hkv, D, pos, cs, sn, rows);
      std::vector<int32_t> start(B, pos), lens(B, pos + S);
      REQUIRE(sai_or_kv_append(k.data(), vs[l].data(), B, S, Hkv, D, start.data(), nullptr, nullptr, 0, 0, 0, 1,
                               T, lay[l].k8.data(), lay[l].v8.data(), lay[l].ks.data(), lay[l].vs.data(), nullptr,
                               nullptr) == 0,
              "oracle append");
      std::vector<float> kd((size_t)B * Hkv * T * D), vd(kd.size());
      REQUIRE(sai_or_kv_dequant(B, Hkv, D, 1, T, lens.data(), lay[l].k8.data(), lay[l].v8.data(), lay[l].ks.data(),
                                lay[l].vs.data(), nullptr, nullptr, kd.data(), vd.data()) == 0,
              "oracle dequant");
      std::vector<float> want((size_t)B * S * Hq * D);
      const bool sliding = l % 2 == 0;
      REQUIRE(sai_or_gqa_cached_window(q.data(), B, S, Hq, Hkv, D, lens.data(), T, kd.data(), vd.data(), nullptr,
                                       nullptr, 0, 0, 0, 0, 0.0f, sliding ? W : 0, sliding ? W : -1,
                                       want.data()) == 0,
              "oracle attention");
      char w[96];
      std::snprintf(w, sizeof w, "%s layer %d", what, l);
      close(host_f32(got[l]), want, w);
    }
    pos += S;
    REQUIRE(session->position() == (size_t)pos, "%s: position %zu", what, session->position());
  };
  pass(40, "prefill pass");
  for (int step = 0; step < 6; ++step) pass(1, "decode pass");
  must(session->reset_kv_cache(), "reset");
  REQUIRE(session->position() == 0, "reset position");
  clear();
  pos = 0;
  pass(9, "pass after reset");
  pass(1, "decode after reset");
  // errors: an op this library does not implement, an output never produced
  std::vector<ExecutionNode> g2 = {{"mm", "MatMul", {"a", "b"}, {"c"}, {}}};
  auto s2 = must(GpuSession::create(0, cfg, g2, {"c"}), "create");
  SessionError e = must_fail_session(s2->run({}), "MatMul");
  REQUIRE(e.to_string() == "execution failed: mm: internal error: GPU executor: no GPU implementation for MatMul",
          "%s", e.to_string().c_str());
  auto s3 = must(GpuSession::create(0, cfg, {}, {"nothing"}), "create");
  e = must_fail_session(s3->run({}), "missing output");
  REQUIRE(e.to_string() == "execution failed: GPU executor: output tensor 'nothing' not produced", "%s",
          e.to_string().c_str());
}

void gpu_session_gemma_graph() { gemma_graph_session(8, 2, 128, 10000.0, 61); }

// A bf16 graph whose attention outputs feed the next layer: layer l's
// RotaryEmbedding takes attn(l-1) as its x. attn_out comes back in Q's
// dtype (bf16, as gpu_gqa returns it, attention.rs:835 and :877-901), which
// is what a bf16 consumer needs: the reference's next op, the bf16 o_proj
// GEMM, takes only bf16 x bf16 (pick_gemm_dtype, gpu_executor.rs:1024-1031),
// and the RotaryEmbedding node here takes it unchanged. Each layer is checked
// against the oracle from the input the GPU actually fed it (the previous
// layer's bf16 output): RoPE bit for bit after rounding to bf16, attention
// within the bf16-widened tolerance, over a prefill pass and decode passes.
void gpu_session_bf16_chain() {
  const int L = 3, B = 2, Hq = 8, Hkv = 2, D = 128, rows = 96, T = 64;
  SessionConfig cfg;
  cfg.num_hidden_layers = L;
  cfg.num_key_value_heads = Hkv;
  cfg.head_dim = D;
  cfg.max_seq_len = T;
  cfg.max_batch = B;
  std::vector<ExecutionNode> graph;
  std::vector<std::string> outs;
  for (int l = 0; l < L; ++l) {
    const std::string i = std::to_string(l);
    const std::string x = l == 0 ? "q0" : "attn" + std::to_string(l - 1);
    graph.push_back({"rope_q" + i, "RotaryEmbedding", {x, "cos", "sin"}, {"qr" + i},
                     {AttributeProto::make_int("rotary_embedding_dim", D), AttributeProto::make_int("interleaved", 0)}});
    graph.push_back({"rope_k" + i, "RotaryEmbedding", {"k" + i, "cos", "sin"}, {"kr" + i},
                     {AttributeProto::make_int("rotary_embedding_dim", D), AttributeProto::make_int("interleaved", 0)}});
    graph.push_back({"gqa" + i, "GroupQueryAttention", {"qr" + i, "kr" + i, "v" + i, "", ""},
                     {"attn" + i, "present_k" + i, "present_v" + i},
                     {AttributeProto::make_int("num_heads", Hq), AttributeProto::make_int("kv_num_heads", Hkv)}});
    outs.push_back("attn" + i);
  }
  auto session = must(GpuSession::create(0, cfg, graph, outs), "GpuSession::create");
  std::vector<float> cs, sn;
  rope_tables(rows, D, 10000.0, cs, sn);
  struct Lay { std::vector<int8_t> k8, v8; std::vector<float> ks, vs; };
  std::vector<Lay> lay(L);
  for (Lay& x : lay) {
    x.k8.assign((size_t)B * Hkv * T * D, 0); x.v8.assign(x.k8.size(), 0);
    x.ks.assign((size_t)B * Hkv * T, 0.0f); x.vs.assign(x.ks.size(), 0.0f);
  }
  auto round_bf16 = [](std::vector<float>& x) {
    for (float& e : x) e = sai_or_bf16_to_f32(sai_or_f32_to_bf16(e));
  };
  std::mt19937_64 gen(63);
  int pos = 0;
  auto pass = [&](int S, const char* what) {
    std::vector<std::pair<std::string, DeviceTensor>> in;
    in.emplace_back("cos", f32_tensor(cs, shp({rows, D / 2})));
    in.emplace_back("sin", f32_tensor(sn, shp({rows, D / 2})));
    std::vector<float> q0 = gauss(gen, (size_t)B * S * Hq * D);
    in.emplace_back("q0", bf16_tensor(q0, shp({B, S, (int64_t)Hq * D})));  // q0: the bf16 values
    std::vector<std::vector<float>> ks(L), vs(L);
    for (int l = 0; l < L; ++l) {
      const std::string i = std::to_string(l);
      ks[l] = gauss(gen, (size_t)B * S * Hkv * D);
      vs[l] = gauss(gen, (size_t)B * S * Hkv * D);
      in.emplace_back("k" + i, bf16_tensor(ks[l], shp({B, S, (int64_t)Hkv * D})));
      in.emplace_back("v" + i, bf16_tensor(vs[l], shp({B, S, (int64_t)Hkv * D})));
    }
    auto got = must(session->run(std::move(in)), what);
    REQUIRE(got.size() == (size_t)L, "%s: outputs", what);
    std::vector<float> x = q0;  // layer l's RoPE input as the GPU saw it
    for (int l = 0; l < L; ++l) {
      REQUIRE(got[l].dtype == DataType::BFloat16, "%s layer %d: attn_out is not bf16", what, l);
      std::vector<float> q = x, k = ks[l];
      oracle_rope_bshd(q, B, S, Hq, D, pos, cs, sn, rows);
      oracle_rope_bshd(k, B, S, Hkv, D, pos, cs, sn, rows);
      round_bf16(q);  // the bf16 RotaryEmbedding outputs the GQA node reads
      round_bf16(k);
      std::vector<int32_t> start(B, pos), lens(B, pos + S);
      REQUIRE(sai_or_kv_append(k.data(), vs[l].data(), B, S, Hkv, D, start.data(), nullptr, nullptr, 0, 0, 0, 1,
                               T, lay[l].k8.data(), lay[l].v8.data(), lay[l].ks.data(), lay[l].vs.data(), nullptr,
                               nullptr) == 0,
              "oracle append");
      std::vector<float> kd((size_t)B * Hkv * T * D), vd(kd.size());
      REQUIRE(sai_or_kv_dequant(B, Hkv, D, 1, T, lens.data(), lay[l].k8.data(), lay[l].v8.data(), lay[l].ks.data(),
                                lay[l].vs.data(), nullptr, nullptr, kd.data(), vd.data()) == 0,
              "oracle dequant");
      std::vector<float> want((size_t)B * S * Hq * D);
      REQUIRE(sai_or_gqa_cached_window(q.data(), B, S, Hq, Hkv, D, lens.data(), T, kd.data(), vd.data(), nullptr,
                                       nullptr, 0, 0, 0, 0, 0.0f, 0, -1, want.data()) == 0,
              "oracle attention");
      const std::vector<float> a = host_values(got[l]);
      char w[96];
      std::snprintf(w, sizeof w, "%s layer %d", what, l);
      close_bf16(a, want, w);
      x = a;  // the next layer's RotaryEmbedding reads this output
    }
    pos += S;
  };
  pass(21, "bf16 chain prefill");
  for (int step = 0; step < 3; ++step) pass(1, "bf16 chain decode");
}

// Gemma 3 4B's attention shape (model_loader/config.rs:695-717): 8 query heads
// over 4 kv heads, head_dim 256, rope_theta 1e6.
void gpu_session_gemma3_head256() { gemma_graph_session(8, 4, 256, 1000000.0, 62); }

// Gemma 4 31B's attention shape (model_loader/config.rs:720-737): 32 query
// heads over 8 kv heads, head_dim 168 (the cache stores it 192 wide),
// rope_theta 1e6; and the CPU op's cache path at head_dim 168.
void gpu_session_gemma4_head168() { gemma_graph_session(32, 8, 168, 1000000.0, 63); }
void gpu_cpu_op_gqa_head168() {
  cpu_op_case(false, 2, 32, 8, 168, 1, 37, true, false, false, 45);   // decode step
  cpu_op_case(false, 1, 32, 8, 168, 40, 70, true, true, false, 46);   // chunk over a past
}

// GpuCompressedKvCache (CompressedKVCache, kv_compression.rs:738-963) with the
// low-rank K on: two sequences x two kv heads, head_dim 128, 4-bit + QJL, a
// 520-row pass (the low-rank state re-decomposes at row 513) and a fused
// one-row step. read_v is bit-exact with the oracle's encode + decode,
// read_k with the oracle's low-rank reconstruction, the attention within
// 2e-3 + 1e-2 relative of the oracle's estimator; errors map to OpError.
void gpu_compressed_kv_cache() {
  const int B = 2, H = 2, D = 128, S = 520, Hq = 4, G = Hq / H, BITS = 4;
  KVCacheConfig cfg;
  cfg.kv_quant_bits = BITS;
  cfg.num_kv_heads = H;
  cfg.head_dim = D;
  cfg.kv_lowrank_k = 4;
  GpuCompressedKvCache c = must(GpuCompressedKvCache::create(runtime(), cfg, B, 600), "create");
  std::mt19937 rng(71);
  std::normal_distribution<float> nd;
  auto randv = [&](size_t n) {
    std::vector<float> v(n);
    for (float& x : v) x = nd(rng);
    return v;
  };
  const std::vector<float> k = randv((size_t)B * S * H * D), v = randv(k.size());
  must(c.write_kv(0, must(DeviceTensor::from_f32(k, shp({B, S, H * D})), "k"),
                  must(DeviceTensor::from_f32(v, shp({B, S, H * D})), "v")), "write_kv");
  must(c.advance(), "advance");
  {
    // shapes that claim more than their buffers hold are rejected
    DeviceTensor short_k = must(DeviceTensor::from_f32(std::vector<float>((size_t)H * D), shp({1, 1, H * D})), "short");
    short_k.shape = shp({B, 1, H * D});
    OpError e = must_fail(c.write_kv(0, short_k, short_k), "write_kv short K");
    REQUIRE(e.kind == OpError::Kind::ShapeMismatch, "%s", e.to_string().c_str());
    DeviceTensor short_q = must(DeviceTensor::from_f32(std::vector<float>((size_t)Hq * D), shp({1, 1, Hq * D})), "short q");
    short_q.shape = shp({B, 1, Hq * D});
    e = must_fail(c.attend(0, short_q, Hq), "attend short Q");
    REQUIRE(e.kind == OpError::Kind::ShapeMismatch, "%s", e.to_string().c_str());
  }
  const std::vector<float> q = randv((size_t)B * Hq * D), k1 = randv((size_t)B * H * D),
                           v1 = randv(k1.size());
  DeviceTensor out = must(c.write_attend(0, must(DeviceTensor::from_f32(q, shp({B, 1, Hq * D})), "q"),
                                         must(DeviceTensor::from_f32(k1, shp({B, 1, H * D})), "k1"),
                                         must(DeviceTensor::from_f32(v1, shp({B, 1, H * D})), "v1"),
                                         Hq), "write_attend");
  must(c.advance(), "advance 2");
  REQUIRE(c.seq_len(0) == S + 1 && c.seq_len(1) == S + 1, "seq_len %zu", c.seq_len(0));
  const std::vector<float> got = must(out.to_host_f32(), "out");
  const int R = S + 1, cb = D * BITS / 8, W = D / 64;
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h) {
      std::vector<int8_t> sg(D);
      sai_or_tq_signs(sai_or_tq_head_seed(cfg.seed, 0, H, h), D, sg.data());
      std::vector<float> kr((size_t)R * D), vr((size_t)R * D);
      for (int t = 0; t < R; ++t)
        for (int d = 0; d < D; ++d) {
          const size_t src = t < S ? (((size_t)b * S + t) * H + h) * D + d : ((size_t)b * H + h) * D + d;
          kr[(size_t)t * D + d] = t < S ? k[src] : k1[src];
          vr[(size_t)t * D + d] = t < S ? v[src] : v1[src];
        }
      std::vector<uint8_t> kc((size_t)R * cb), vc((size_t)R * cb);
      std::vector<float> ks(R), kz(R), kcm(R), vs(R), vz(R), vcm(R);
      std::vector<uint64_t> ksb((size_t)R * W), vsb((size_t)R * W);
      for (int t = 0; t < R; ++t) {
        REQUIRE(sai_or_tq_write_row(&kr[(size_t)t * D], D, BITS, sg.data(), 1, &kc[(size_t)t * cb],
                                    &ks[t], &kz[t], &ksb[(size_t)t * W], &kcm[t]) == 0, "k row");
        REQUIRE(sai_or_tq_write_row(&vr[(size_t)t * D], D, BITS, sg.data(), 1, &vc[(size_t)t * cb],
                                    &vs[t], &vz[t], &vsb[(size_t)t * W], &vcm[t]) == 0, "v row");
      }
      // read_v: rows 500 .. 520, bit for bit
      const std::vector<float> gv = must(c.read_v(0, b, h, 500, R - 500), "read_v");
      std::vector<float> want(D);
      for (int t = 500; t < R; ++t) {
        sai_or_tq_decode(&vc[(size_t)t * cb], D, BITS, vs[t], vz[t], sg.data(), want.data());
        REQUIRE(std::memcmp(&gv[(size_t)(t - 500) * D], want.data(), D * 4) == 0, "read_v row %d", t);
      }
      // read_k: the low-rank reconstruction, bit for bit
      std::vector<float> us(R), vt(D);
      int rows = 1, rank = sai_or_lr_decompose(kr.data(), 1, D, 4, us.data(), vt.data()), wc = 0;
      REQUIRE(rank == 1, "rank %d", rank);
      for (int t = 1; t < R; ++t)
        sai_or_lr_update(us.data(), vt.data(), &rows, D, &rank, &wc, &kr[(size_t)t * D]);
      std::vector<float> rec((size_t)R * D);
      sai_or_lr_reconstruct(us.data(), vt.data(), R, D, rank, rec.data());
      const std::vector<float> gk = must(c.read_k(0, b, h, 500, R - 500), "read_k");
      REQUIRE(std::memcmp(gk.data(), &rec[(size_t)500 * D], gk.size() * 4) == 0, "read_k b%d h%d", b, h);
      // the fused step's attention for this kv head's query heads
      std::vector<float> wo((size_t)G * D);
      REQUIRE(sai_or_tq_attend(&q[((size_t)b * Hq + h * G) * D], G, D, BITS, 1, sg.data(), R,
                               kc.data(), ks.data(), kz.data(), ksb.data(), kcm.data(), vc.data(),
                               vs.data(), vz.data(), 1.0f / std::sqrt((float)D), wo.data()) == 0,
              "oracle attend");
      for (int i = 0; i < G * D; ++i) {
        const float g = got[((size_t)b * Hq + h * G) * D + i], w = wo[i];
        REQUIRE(std::fabs(g - w) <= 2e-3f + 1e-2f * std::fabs(w), "attend b%d h%d i%d %g vs %g", b,
                h, i, g, w);
      }
    }
  // reference accounting: blocks + residuals per row, plus the low-rank state
  const size_t per_row = 2 * (cb + 25) + 2 * (W * 8 + 12);
  const size_t want_bytes = (size_t)B * R * H * per_row + (size_t)B * H * (R * 4 + D * 4 + 32);
  REQUIRE(c.memory_bytes() == want_bytes, "memory_bytes %zu vs %zu", c.memory_bytes(), want_bytes);
  KVCacheConfig bad = cfg;
  bad.kv_quant_bits = 5;
  OpError e = must_fail(GpuCompressedKvCache::create(runtime(), bad, 1, 8), "bits 5");
  REQUIRE(e.kind == OpError::Kind::InvalidAttribute, "kind");
  bad = cfg;
  bad.head_dim = 96;
  e = must_fail(GpuCompressedKvCache::create(runtime(), bad, 1, 8), "head_dim 96");
  REQUIRE(e.kind == OpError::Kind::UnsupportedOp, "kind");
  e = must_fail(c.write_kv(0, must(DeviceTensor::from_f32(k1, shp({B, H * D})), "k2"),
                           must(DeviceTensor::from_f32(v1, shp({B, H * D})), "v2")), "rank-2 K");
  REQUIRE(e.kind == OpError::Kind::ShapeMismatch, "kind");
}

// test_kv_cache_sliding_window (tests/test_cuda.rs:1275-1334): a global layer
// and a sliding-window layer of 4; after 6 tokens the global view holds 6,
// the local view the last 4 (positions 2..5), read back by value.
void gpu_cache_sliding_window() {
  RocmRuntime& rt = runtime();
  const size_t Hkv = 2, D = 64;
  GpuKvCache cache = must(GpuKvCache::allocate(rt, 2, Hkv, D, 16, KvQuant::Int8,
                                               {LayerKind::global(), LayerKind::sliding_window(4)}),
                          "allocate");
  for (int pos = 0; pos < 6; ++pos) {
    const float fill = (float)(pos + 1) * 0.1f;
    DeviceTensor kv = fill_tensor(Hkv, D, fill);
    for (size_t layer = 0; layer < 2; ++layer) must(cache.append(layer, kv, kv), "append");
    must(cache.advance_position(), "advance");
  }
  REQUIRE(cache.current_position() == 6, "position");
  KvView g = must(cache.view(0), "view global");
  REQUIRE(g.start_token == 0 && g.token_count == 6, "global view %zu+%zu", g.start_token, g.token_count);
  KvView l = must(cache.view(1), "view local");
  REQUIRE(l.start_token == 2 && l.token_count == 4, "local view %zu+%zu", l.start_token, l.token_count);
  for (size_t h = 0; h < Hkv; ++h) {
    auto kv = must(cache.read_dequantized(1, 0, h, l.start_token, l.token_count), "read local");
    for (size_t vp = 0; vp < 4; ++vp) {
      const float expect = (float)(vp + 2 + 1) * 0.1f;
      for (size_t d = 0; d < D; ++d)
        REQUIRE(std::fabs(kv.first[vp * D + d] - expect) < 1e-2f, "local pos %zu: %g != %g", vp,
                kv.first[vp * D + d], expect);
    }
  }
  KvView lp = must(cache.view_pending(1), "view_pending local");
  REQUIRE(lp.start_token == 2 && lp.token_count == 4, "nothing pending: same view");
}

int main(int argc, char** argv) {
  struct Case {
    const char* name;
    bool gpu;
    std::function<void()> fn;
  };
  const std::vector<Case> cases = {
      {"gpu_compressed_kv_cache", true, gpu_compressed_kv_cache},
      {"cpu_attrs", false, cpu_attrs},
      {"cpu_validate", false, cpu_validate},
      {"cpu_errors_and_types", false, cpu_errors_and_types},
      {"cpu_layer_kinds_for_gemma", false, cpu_layer_kinds_for_gemma},
      {"gpu_cache_allocate_and_append", true, gpu_cache_allocate_and_append},
      {"gpu_cache_multiple_tokens", true, gpu_cache_multiple_tokens},
      {"gpu_cache_reset", true, gpu_cache_reset},
      {"gpu_cache_errors", true, gpu_cache_errors},
      {"gpu_gqa_with_cache_first_token", true, gpu_gqa_with_cache_first_token},
      {"gpu_gqa_first_token_no_history", true, gpu_gqa_first_token_no_history},
      {"gpu_dispatch_errors", true, gpu_dispatch_errors},
      {"gpu_dispatch_rope_tables", true, gpu_dispatch_rope_tables},
      {"gpu_rotary_cpu_op_kats", true, gpu_rotary_cpu_op_kats},
      {"gpu_rotary_dispatch", true, gpu_rotary_dispatch},
      {"gpu_rope_tables", true, gpu_rope_tables},
      {"gpu_session_int8_prefill_decode", true, gpu_session_int8_prefill_decode},
      {"gpu_session_int8_bf16_d64", true, gpu_session_int8_bf16_d64},
      {"gpu_session_int4_decode", true, gpu_session_int4_decode},
      {"gpu_session_int4_bf16_group4", true, gpu_session_int4_bf16_group4},
      {"gpu_session_int4_prefill_decode", true, gpu_session_int4_prefill_decode},
      {"gpu_session_int8_windows", true, gpu_session_int8_windows},
      {"gpu_session_int4_layer_window", true, gpu_session_int4_layer_window},
      {"gpu_cache_sliding_window", true, gpu_cache_sliding_window},
      {"gpu_cpu_op_gqa_with_past", true, gpu_cpu_op_gqa_with_past},
      {"gpu_cpu_op_mha_with_past", true, gpu_cpu_op_mha_with_past},
      {"gpu_cpu_op_kats", true, gpu_cpu_op_kats},
      {"gpu_session_gemma_graph", true, gpu_session_gemma_graph},
      {"gpu_session_bf16_chain", true, gpu_session_bf16_chain},
      {"gpu_session_gemma3_head256", true, gpu_session_gemma3_head256},
      {"gpu_session_gemma4_head168", true, gpu_session_gemma4_head168},
      {"gpu_cpu_op_gqa_head168", true, gpu_cpu_op_gqa_head168},
  };
  std::vector<const Case*> run;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    for (const Case& c : cases)
      if ((a == "--cpu" && !c.gpu) || (a == "--gpu" && c.gpu) || a == c.name) run.push_back(&c);
  }
  if (run.empty()) {
    for (const Case& c : cases) std::printf("%s%s\n", c.name, c.gpu ? " (gpu)" : "");
    return argc > 1 ? 1 : 0;
  }
  int failed = 0;
  for (const Case* c : run) {
    std::printf("RUN  %s\n", c->name);
    std::fflush(stdout);
    try {
      c->fn();
      std::printf("PASS %s\n", c->name);
    } catch (const Failure& f) {
      std::printf("FAIL %s: %s\n", c->name, f.msg.c_str());
      ++failed;
    }
    std::fflush(stdout);
  }
  std::printf("%d of %zu cases failed\n", failed, run.size());
  return failed;
}
