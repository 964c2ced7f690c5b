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
#include <random>
#include <string>
#include <vector>

#include "../../oracle/sai_oracle.h"
#include "../../smallaios_amd/host/gqa_host.hpp"

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
  REQUIRE(!RocmRuntime::supports_op("MatMul") && !RocmRuntime::supports_op(""), "only GQA");
  REQUIRE(element_size(DataType::Float) == 4 && element_size(DataType::BFloat16) == 2 &&
              element_size(DataType::Int64) == 8 && element_size(DataType::Int8) == 1,
          "element sizes");
  DeviceTensor t;
  t.shape = shp({2, -1, 3});
  REQUIRE(t.total_elements() == 0 && t.byte_size() == 0, "negative dim");
  t.shape = shp({2, 3, 4});
  t.dtype = DataType::BFloat16;
  REQUIRE(t.total_elements() == 24 && t.byte_size() == 48, "sizes");
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
                                                   {LayerKind::sliding_window(4)}),
                              "window")) == "kv_cache_allocate:sliding_window", "sliding_window");
  REQUIRE(op_of(must_fail_hip(GpuKvCache::allocate(rt, 1, 2, 16, 8, KvQuant::Int8, {LayerKind::global()}),
                              "head_dim")) == "kv_cache_allocate:unsupported_head_dim", "head_dim");
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
  std::vector<AttributeProto> win = heads;
  win.push_back(AttributeProto::make_int("local_window_size", 4));
  expect(dispatch_gqa(rt, {&q, &k, &k}, win, nullptr), OpError::Kind::InvalidAttribute,
         "local_window_size != -1 not supported", "window");
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
// appends into a logical cache and attends over its dequantised contents.
static void session(KvQuant quant, bool bf16, int B, int Hq, int Hkv, int D, int prefill,
                    int steps, unsigned seed) {
  RocmRuntime& rt = runtime();
  const int layers = 2, rows = 512, t_cap = prefill + steps;
  std::vector<float> cs, sn;
  rope_tables(rows, D, 10000.0, cs, sn);
  DeviceTensor dcos = f32_tensor(cs, shp({rows, D / 2})), dsin = f32_tensor(sn, shp({rows, D / 2}));
  GpuKvCache cache = must(GpuKvCache::allocate(rt, layers, Hkv, D, t_cap, quant,
                                               std::vector<LayerKind>(layers, LayerKind::global()), B),
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
  const std::vector<AttributeProto> attrs = {AttributeProto::make_int("num_heads", Hq),
                                             AttributeProto::make_int("kv_num_heads", Hkv)};
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
      std::vector<float> got = must(outs[0].to_host_f32(), "download");
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
      REQUIRE(sai_or_gqa_cached(q.data(), B, S, Hq, Hkv, D, lens.data(), t_cap, kd.data(), vd.data(),
                                cs.data(), sn.data(), rows, 1, 0, 0, 0.0f, want.data()) == 0,
              "oracle gqa");
      char what[96];
      std::snprintf(what, sizeof what, "pass %d layer %d output", pass, layer);
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

int main(int argc, char** argv) {
  struct Case {
    const char* name;
    bool gpu;
    std::function<void()> fn;
  };
  const std::vector<Case> cases = {
      {"cpu_attrs", false, cpu_attrs},
      {"cpu_validate", false, cpu_validate},
      {"cpu_errors_and_types", false, cpu_errors_and_types},
      {"gpu_cache_allocate_and_append", true, gpu_cache_allocate_and_append},
      {"gpu_cache_multiple_tokens", true, gpu_cache_multiple_tokens},
      {"gpu_cache_reset", true, gpu_cache_reset},
      {"gpu_cache_errors", true, gpu_cache_errors},
      {"gpu_gqa_with_cache_first_token", true, gpu_gqa_with_cache_first_token},
      {"gpu_gqa_first_token_no_history", true, gpu_gqa_first_token_no_history},
      {"gpu_dispatch_errors", true, gpu_dispatch_errors},
      {"gpu_dispatch_rope_tables", true, gpu_dispatch_rope_tables},
      {"gpu_session_int8_prefill_decode", true, gpu_session_int8_prefill_decode},
      {"gpu_session_int8_bf16_d64", true, gpu_session_int8_bf16_d64},
      {"gpu_session_int4_decode", true, gpu_session_int4_decode},
      {"gpu_session_int4_bf16_group4", true, gpu_session_int4_bf16_group4},
      {"gpu_session_int4_prefill_decode", true, gpu_session_int4_prefill_decode},
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
