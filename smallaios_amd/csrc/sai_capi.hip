// C ABI of libsai_hip (declared in include/sai_hip.h).
//
// Host-side responsibilities: argument and shape validation with the
// reference's error kinds, the host mirror of page table and lengths (every
// page id and position a kernel will touch is checked here before launch),
// workspace management and kernel dispatch. No exception leaves this file.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/sai_hip.h"
#include "sai_internal.h"

#define SAI_API extern "C" __attribute__((visibility("default")))

struct sai_ctx {
  int device = 0;
  int num_cus = 0;
  std::string err;
  int32_t decode_split = 0;  // 0 = automatic
  int32_t tq_split = 0;      // TurboQuant attention split, positions (0 = automatic)
  int32_t decode_waves = 0;  // 0: automatic
  int32_t decode_merge = 2;  // 0: combine kernel, 1: in-kernel merge, 2: automatic
  // tile order of the int8 decode and the TurboQuant attention: 1 fixed in
  // both (bit-reproducible), 0 handed out at run time in both, 2 fixed in
  // the int8 decode only (measured ~0.5 % slower there at 16 x 8k, but 6-10 %
  // slower in the TurboQuant attention)
  int32_t reproducible = 2;
  int32_t last_wg = 0;
  int32_t last_split = 0;
  int32_t last_launches = 0;  // kernels of the last decode call (decode, + combine)
  // decode-kernel timing ring: event pairs of the last `slots` calls
  std::vector<hipEvent_t> ev_start, ev_end;
  int64_t timed_calls = 0;
};

// Device scratch of the decode kernels: split partials (m, l, o), per-sequence
// split ranges for the combine kernel, and the in-kernel merge's ticket
// counters (zero between launches: each launch's last workgroup resets its
// counter). Each cache owns one, sized when the cache is created, so that
// caches used from different streams never share one.
struct DecodeWorkspace {
  float* partials = nullptr;
  size_t partial_floats = 0;
  int32_t* seq_info = nullptr;
  size_t seq_info_n = 0;
  int32_t* counters = nullptr;
  size_t counter_n = 0;
  // prefill: one large-V flag per workgroup (zero between launches: the
  // precise pass clears what the fast pass set)
  int32_t* prec_flags = nullptr;
  size_t prec_flags_n = 0;
};

// Scratch of sai_gqa_with_cache_noalloc, for callers that cannot allocate
// device memory: one fixed array per GPU, held until the process ends,
// holding the same three parts as a DecodeWorkspace (merge ticket counters,
// split ranges, split partials, in that order). Its device address on each
// GPU is taken once, in sai_init, with that GPU current (g_scratch below);
// host code never passes `scratch` itself to a kernel (on the host that name
// is only a stand-in for the symbol).
constexpr size_t kScratchBytes = (size_t)16 << 20;
constexpr size_t kScratchCounters = 65536;  // int32: sequences x kv heads
constexpr size_t kScratchSeqInfo = 65536;   // int32: two per sequence
constexpr size_t kScratchPartialFloats =
    (kScratchBytes - sizeof(int32_t) * (kScratchCounters + kScratchSeqInfo)) / sizeof(float);
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// Per device: the scratch's device address (0 until sai_init has set it up
// on that device) and whether that set-up failed.
constexpr int kMaxScratchDevices = 64;
struct ScratchSlot {
  void* ptr = nullptr;
  bool failed = false;
};
std::mutex g_scratch_mu;
ScratchSlot g_scratch[kMaxScratchDevices];

struct sai_tqcache {
  sai_tqcache_desc desc{};
  size_t code_stride = 0;  // bytes of one row's K codes, multiple of 16
  size_t rows_total = 0;   // heads * max_batch * max_rows
  int32_t tiles_cap = 0;   // 64-position V tiles per (head, sequence)
  struct Layer {
    uint8_t* codes_k = nullptr;
    uint8_t* codes_v = nullptr;
    float4* par_k = nullptr;
    float4* par_v = nullptr;
    uint32_t* sg_k = nullptr;
    uint32_t* sg_v = nullptr;
    int8_t* rot = nullptr;  // rotation signs [heads][D]
    float* lr_us = nullptr;  // low-rank K: U_S per row, Vt, u scratch
    float* lr_vt = nullptr;
    float* lr_u = nullptr;
    bool lr_written = false;  // its low-rank state took this pass's rows
  };
  std::vector<Layer> layers;
  int32_t* d_lens = nullptr;
  std::vector<int32_t> h_lens;
  int32_t batch = 0;
  int32_t pending = 0;
  float norm = 0.0f;
  // attention split partials, sized at creation, and the split tickets of
  // each (sequence, kv head) (zero between launches: the workgroup that takes
  // the last ticket resets it)
  float* partials = nullptr;
  size_t partial_floats = 0;
  int32_t* counters = nullptr;
};

struct sai_kvcache {
  sai_kvcache_desc desc{};
  size_t block_bytes = 0;
  size_t pool_bytes = 0;
  std::vector<uint8_t*> pools;
  int32_t* d_page_table = nullptr;
  int32_t* d_seq_lens = nullptr;
  std::vector<int32_t> h_page_table;  // [max_batch][max_pages_per_seq]
  std::vector<int32_t> h_mapped;      // leading mapped pages per sequence
  std::vector<int32_t> h_seq_lens;    // committed
  int32_t batch = 0;
  int32_t pending = 0;
  std::vector<int32_t> layer_window;  // per layer: last keys visible (0: global)
  DecodeWorkspace ws;
};

namespace {

sai_status fail(sai_ctx* ctx, sai_status code, const char* fmt, ...) {
  if (ctx) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    ctx->err = buf;
  }
  return code;
}

sai_status hip_fail(sai_ctx* ctx, hipError_t e, const char* what) {
  return fail(ctx, SAI_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// Newton square root of the reference (onnx-rt/src/ops/microsoft.rs:54-63);
// the default GQA scale is 1 / sqrt_f32(head_dim) (microsoft.rs:1153).
float sqrt_f32_newton(float x) {
  if (x <= 0.0f) return 0.0f;
  volatile float guess = x;  // keep every step in f32, unfused
  for (int i = 0; i < 16; ++i) {
    volatile float q = x / guess;
    volatile float s = guess + q;
    guess = 0.5f * s;
  }
  return guess;
}

// Largest decode split (the kernel stages a split's page ids in LDS).
constexpr int32_t kMaxDecodeSplit = 16384;

// int8 and int4: head_dim 64, 128 and 256 (Gemma 3); int8 also 168 (Gemma 4
// 31B), stored as 192 (sai::stored_head_dim). int4's groups of 32 do not
// divide 168.
bool supported_dims(int head_dim, int quant) {
  if (quant == SAI_KV_INT8 || quant == SAI_KV_INT4)
    return head_dim == 64 || head_dim == 128 || head_dim == 256 ||
           (head_dim == 168 && quant == SAI_KV_INT8);
  return false;
}

struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) == hipSuccess && prev != dev) (void)hipSetDevice(dev);
  }
  ~DeviceGuard() {
    int cur;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

// Common checks before a kernel touches the pages of positions [0, len_b).
sai_status check_lengths(sai_ctx* ctx, const sai_kvcache* c, int32_t batch, int32_t extra,
                         const char* op) {
  if (batch <= 0 || batch != c->batch)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH,
                "%s: batch %d does not match the cache's page table batch %d", op, batch,
                c->batch);
  const int64_t cap = (int64_t)c->desc.max_pages_per_seq * SAI_PAGE_TOKENS;
  for (int i = 0; i < batch; ++i) {
    const int64_t len = (int64_t)c->h_seq_lens[i] + extra;
    if (len > cap)
      return fail(ctx, SAI_ERR_OVERFLOW, "%s: position_overflow (sequence %d needs %lld > %lld)",
                  op, i, (long long)len, (long long)cap);
    const int64_t pages = (len + SAI_PAGE_TOKENS - 1) / SAI_PAGE_TOKENS;
    if (pages > c->h_mapped[i])
      return fail(ctx, SAI_ERR_SHAPE_MISMATCH,
                  "%s: sequence %d needs %lld pages but only %d leading pages are mapped", op, i,
                  (long long)pages, c->h_mapped[i]);
  }
  return SAI_OK;
}

sai_status check_rope(sai_ctx* ctx, const sai_kvcache* c, int32_t batch, int32_t extra,
                      const float* cos_cache, const float* sin_cache, int32_t cache_rows,
                      int32_t do_rotary, const char* op) {
  if (!do_rotary) return SAI_OK;
  if (!cos_cache || !sin_cache)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "%s: do_rotary=1 but cos_cache/sin_cache is missing",
                op);
  // the kernels read a table row in 16-byte pieces
  if ((((uintptr_t)cos_cache | (uintptr_t)sin_cache) & 15u) != 0)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "%s: cos_cache/sin_cache must be 16-byte aligned",
                op);
  int32_t maxlen = 0;
  for (int i = 0; i < batch; ++i) maxlen = std::max(maxlen, c->h_seq_lens[i] + extra);
  if (maxlen > cache_rows)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "%s: position %d out of cache range %d", op,
                maxlen - 1, cache_rows);
  return SAI_OK;
}

// Keys visible to a query (0: all): the cache layer's window keeps the last
// layer_window keys (GpuKvCache::view_at, kv_cache.rs:340-360); the node's
// window hides keys before q_pos - window, which leaves window + 1
// (gqa_softmax_mask_f32, cuda/kernels/attention.rs:79). Both: the narrower.
int32_t visible_span(int32_t layer_window, int32_t window) {
  int64_t w = layer_window > 0 ? layer_window : 0;
  if (window > 0) {
    const int64_t m = (int64_t)window + 1;
    if (w == 0 || m < w) w = m;
  }
  return (int32_t)std::min<int64_t>(w, 0x7FFFFFFF);
}

void release_workspace(DecodeWorkspace& w) {
  if (w.partials) (void)hipFree(w.partials);
  if (w.seq_info) (void)hipFree(w.seq_info);
  if (w.counters) (void)hipFree(w.counters);
  if (w.prec_flags) (void)hipFree(w.prec_flags);
  w = DecodeWorkspace{};
}

// Grows the prefill flags to n (zeroed, after the device is idle).
sai_status reserve_prec_flags(sai_ctx* ctx, DecodeWorkspace& w, size_t n) {
  if (n <= w.prec_flags_n) return SAI_OK;
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(ctx, e, "prefill flags: sync");
  if (w.prec_flags) (void)hipFree(w.prec_flags);
  w.prec_flags = nullptr;
  w.prec_flags_n = 0;
  e = hipMalloc(&w.prec_flags, n * sizeof(int32_t));
  if (e != hipSuccess) return fail(ctx, SAI_ERR_ALLOC, "prefill flags: %s", hipGetErrorString(e));
  e = hipMemset(w.prec_flags, 0, n * sizeof(int32_t));
  if (e != hipSuccess) return hip_fail(ctx, e, "prefill flags memset");
  e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(ctx, e, "prefill flags: sync");
  w.prec_flags_n = n;
  return SAI_OK;
}

// Grows w to hold at least the given sizes. A buffer that must grow is freed
// and allocated again after the device is idle (no launch still uses it);
// counters start at zero.
sai_status reserve_workspace(sai_ctx* ctx, DecodeWorkspace& w, size_t partial_floats,
                             size_t seq_info, size_t counters) {
  if (partial_floats <= w.partial_floats && seq_info <= w.seq_info_n && counters <= w.counter_n)
    return SAI_OK;
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(ctx, e, "decode workspace: sync");
  if (counters > w.counter_n) {
    if (w.counters) (void)hipFree(w.counters);
    w.counters = nullptr;
    w.counter_n = 0;
    e = hipMalloc(&w.counters, counters * sizeof(int32_t));
    if (e != hipSuccess) return fail(ctx, SAI_ERR_ALLOC, "decode counters: %s", hipGetErrorString(e));
    e = hipMemset(w.counters, 0, counters * sizeof(int32_t));
    if (e != hipSuccess) return hip_fail(ctx, e, "decode counters memset");
    w.counter_n = counters;
  }
  if (partial_floats > w.partial_floats) {
    if (w.partials) (void)hipFree(w.partials);
    w.partials = nullptr;
    w.partial_floats = 0;
    e = hipMalloc(&w.partials, partial_floats * sizeof(float));
    if (e != hipSuccess) return fail(ctx, SAI_ERR_ALLOC, "decode workspace: %s", hipGetErrorString(e));
    w.partial_floats = partial_floats;
  }
  if (seq_info > w.seq_info_n) {
    if (w.seq_info) (void)hipFree(w.seq_info);
    w.seq_info = nullptr;
    w.seq_info_n = 0;
    e = hipMalloc(&w.seq_info, seq_info * sizeof(int32_t));
    if (e != hipSuccess) return fail(ctx, SAI_ERR_ALLOC, "decode sequence info: %s", hipGetErrorString(e));
    w.seq_info_n = seq_info;
  }
  return SAI_OK;
}

// (sequence, split) work items one decode launch can have at the automatic
// split (decode_split_tokens): the split is at least 256 tokens and at least
// (tokens x kv heads) / CUs, except for ragged batches, where it may be capped
// at 3072; so the items number at most CUs / kv heads, or total tokens / 2048
// (a bound with room), plus one rounding item per sequence. Total tokens are bounded by the pages
// (unless sequences share pages; a launch that needs more grows the workspace).
size_t decode_work_bound(const sai_ctx* ctx, const sai_kvcache_desc& d) {
  const size_t by_cus = ((size_t)ctx->num_cus + d.num_kv_heads - 1) / d.num_kv_heads + 1;
  const size_t by_pages = ((size_t)d.num_pages * SAI_PAGE_TOKENS + 2047) / 2048;
  return std::max(by_cus, by_pages) + (size_t)d.max_batch;
}

// Largest query group a cache of this head_dim serves in decode.
// (int8 decodes groups up to 8 at every head dim; int4 at head_dim 256 up to 4)
int max_decode_group(int head_dim, int quant) {
  return head_dim > 128 && quant == SAI_KV_INT4 ? 4 : 8;
}

}  // namespace

// ---------------------------------------------------------------- runtime ---
SAI_API sai_status sai_init(int device, sai_ctx** out) {
  if (!out) return SAI_ERR_NULL;
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return SAI_ERR_HIP;
  sai_ctx* ctx = new (std::nothrow) sai_ctx();
  if (!ctx) return SAI_ERR_ALLOC;
  ctx->device = device;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) == hipSuccess) ctx->num_cus = prop.multiProcessorCount;
  if (ctx->num_cus <= 0) ctx->num_cus = 256;
  // the no-allocation scratch of this device: its address, once, with the
  // device current; its ticket counters must start at zero (every launch
  // that merges in-kernel leaves them at zero again)
  if (device < kMaxScratchDevices) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    ScratchSlot& sl = g_scratch[device];
    if (!sl.ptr && !sl.failed) {
      DeviceGuard dg(device);
      void* ptr = nullptr;
      hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (e == hipSuccess && ptr)
        e = hipMemset(ptr, 0, kScratchCounters * sizeof(int32_t));
      if (e == hipSuccess) e = hipDeviceSynchronize();
      if (e == hipSuccess && ptr)
        sl.ptr = ptr;
      else
        sl.failed = true;
    }
  }
  *out = ctx;
  return SAI_OK;
}

SAI_API void sai_destroy(sai_ctx* ctx) {
  if (!ctx) return;
  DeviceGuard dg(ctx->device);
  for (hipEvent_t e : ctx->ev_start) (void)hipEventDestroy(e);
  for (hipEvent_t e : ctx->ev_end) (void)hipEventDestroy(e);
  delete ctx;
}

SAI_API const char* sai_last_error(const sai_ctx* ctx) { return ctx ? ctx->err.c_str() : ""; }

SAI_API float sai_default_scale(int32_t head_dim) {
  return 1.0f / sqrt_f32_newton((float)head_dim);
}

SAI_API int32_t sai_device_supported(int device) {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return 0;
  return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

SAI_API int32_t sai_set_decode_split(sai_ctx* ctx, int32_t tokens) {
  if (!ctx) return 0;
  int32_t prev = ctx->decode_split;
  if (tokens >= 0 && tokens % 64 == 0 && tokens <= kMaxDecodeSplit) ctx->decode_split = tokens;
  return prev;
}

SAI_API int32_t sai_set_tq_split(sai_ctx* ctx, int32_t rows) {
  if (!ctx) return 0;
  int32_t prev = ctx->tq_split;
  if (rows == 0 || (rows >= 256 && rows % 256 == 0 && rows <= 65536)) ctx->tq_split = rows;
  return prev;
}

SAI_API int32_t sai_set_decode_waves(sai_ctx* ctx, int32_t waves) {
  if (!ctx) return 0;
  int32_t prev = ctx->decode_waves;
  if (waves == 0 || waves == 4 || waves == 8) ctx->decode_waves = waves;
  return prev;
}

SAI_API int32_t sai_set_decode_merge(sai_ctx* ctx, int32_t in_kernel) {
  if (!ctx) return 0;
  int32_t prev = ctx->decode_merge;
  if (in_kernel >= 0 && in_kernel <= 2) ctx->decode_merge = in_kernel;
  return prev;
}

SAI_API int32_t sai_set_decode_reproducible(sai_ctx* ctx, int32_t mode) {
  if (!ctx) return -1;
  const int32_t prev = ctx->reproducible;
  if (mode >= 0 && mode <= 2) ctx->reproducible = mode;
  return prev;
}

SAI_API int32_t sai_set_decode_timing(sai_ctx* ctx, int32_t slots) {
  if (!ctx) return 0;
  const int32_t prev = (int32_t)ctx->ev_start.size();
  DeviceGuard dg(ctx->device);
  for (hipEvent_t e : ctx->ev_start) (void)hipEventDestroy(e);
  for (hipEvent_t e : ctx->ev_end) (void)hipEventDestroy(e);
  ctx->ev_start.clear();
  ctx->ev_end.clear();
  ctx->timed_calls = 0;
  const int32_t n = std::min<int32_t>(std::max<int32_t>(slots, 0), 4096);
  for (int32_t i = 0; i < n; ++i) {
    hipEvent_t a = nullptr, b = nullptr;
    if (hipEventCreate(&a) != hipSuccess) break;
    if (hipEventCreate(&b) != hipSuccess) {
      (void)hipEventDestroy(a);
      break;
    }
    ctx->ev_start.push_back(a);
    ctx->ev_end.push_back(b);
  }
  return prev;
}

SAI_API int32_t sai_decode_kernel_times(sai_ctx* ctx, float* us, int32_t max_n) {
  if (!ctx || !us) return SAI_ERR_NULL;
  const int64_t slots = (int64_t)ctx->ev_start.size();
  if (slots == 0 || ctx->timed_calls == 0 || max_n <= 0) return 0;
  DeviceGuard dg(ctx->device);
  const int64_t n = std::min<int64_t>({(int64_t)max_n, slots, ctx->timed_calls});
  const int64_t last = (ctx->timed_calls - 1) % slots;
  hipError_t e = hipEventSynchronize(ctx->ev_end[last]);
  if (e != hipSuccess) return hip_fail(ctx, e, "decode timing");
  for (int64_t i = 0; i < n; ++i) {
    const int64_t k = (ctx->timed_calls - n + i) % slots;
    float ms = 0.0f;
    e = hipEventElapsedTime(&ms, ctx->ev_start[k], ctx->ev_end[k]);
    if (e != hipSuccess) return hip_fail(ctx, e, "decode timing");
    us[i] = ms * 1000.0f;
  }
  return (int32_t)n;
}

SAI_API sai_status sai_last_decode_shape(const sai_ctx* ctx, int32_t* workgroups,
                                         int32_t* split_tokens) {
  if (!ctx) return SAI_ERR_NULL;
  if (workgroups) *workgroups = ctx->last_wg;
  if (split_tokens) *split_tokens = ctx->last_split;
  return SAI_OK;
}

SAI_API int32_t sai_last_decode_launches(const sai_ctx* ctx) {
  return ctx ? ctx->last_launches : 0;
}

// ------------------------------------------------------------------ cache ---
SAI_API sai_status sai_kvcache_create(sai_ctx* ctx, const sai_kvcache_desc* desc,
                                      sai_kvcache** out) {
  if (!ctx || !desc || !out) return SAI_ERR_NULL;
  *out = nullptr;
  const sai_kvcache_desc& d = *desc;
  if (d.num_layers <= 0 || d.num_kv_heads <= 0 || d.head_dim <= 0 || d.num_pages <= 0 ||
      d.max_batch <= 0 || d.max_pages_per_seq <= 0)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "kv_cache_allocate: zero_dim");
  if (!supported_dims(d.head_dim, d.quant))
    return fail(ctx, SAI_ERR_UNSUPPORTED, "kv_cache_allocate: head_dim %d / quant %d unsupported",
                d.head_dim, d.quant);
  DeviceGuard dg(ctx->device);
  sai_kvcache* c = new (std::nothrow) sai_kvcache();
  if (!c) return fail(ctx, SAI_ERR_ALLOC, "kv_cache_allocate: host");
  c->desc = d;
  const int ds = sai::stored_head_dim(d.head_dim);
  c->block_bytes = d.quant == SAI_KV_INT8 ? sai::block_bytes_int8(ds) : sai::block_bytes_int4(ds);
  c->pool_bytes = (size_t)d.num_pages * d.num_kv_heads * c->block_bytes;
  c->pools.assign(d.num_layers, nullptr);
  hipError_t e = hipSuccess;
  for (int l = 0; l < d.num_layers && e == hipSuccess; ++l) {
    e = hipMalloc(&c->pools[l], c->pool_bytes);
    if (e == hipSuccess) e = hipMemset(c->pools[l], 0, c->pool_bytes);
  }
  const size_t pt_n = (size_t)d.max_batch * d.max_pages_per_seq;
  if (e == hipSuccess) e = hipMalloc(&c->d_page_table, pt_n * sizeof(int32_t));
  if (e == hipSuccess) e = hipMemset(c->d_page_table, 0, pt_n * sizeof(int32_t));
  if (e == hipSuccess) e = hipMalloc(&c->d_seq_lens, (size_t)d.max_batch * sizeof(int32_t));
  if (e == hipSuccess) e = hipMemset(c->d_seq_lens, 0, (size_t)d.max_batch * sizeof(int32_t));
  if (e != hipSuccess) {
    sai_kvcache_destroy(c);
    return fail(ctx, SAI_ERR_ALLOC, "kv_cache_allocate: %s", hipGetErrorString(e));
  }
  c->h_page_table.assign(pt_n, -1);
  c->h_mapped.assign(d.max_batch, 0);
  c->h_seq_lens.assign(d.max_batch, 0);
  c->layer_window.assign(d.num_layers, 0);
  // the decode workspace for every launch at the automatic split
  const size_t work = decode_work_bound(ctx, d);
  sai_status st = reserve_workspace(
      ctx, c->ws, work * d.num_kv_heads * max_decode_group(d.head_dim, d.quant) * (ds + 2),
      (size_t)d.max_batch * 2, (size_t)d.max_batch * d.num_kv_heads);
  if (st != SAI_OK) {
    sai_kvcache_destroy(c);
    return st;
  }
  *out = c;
  return SAI_OK;
}

SAI_API sai_status sai_kvcache_set_layer_window(sai_ctx* ctx, sai_kvcache* c, int32_t layer,
                                                int32_t window) {
  if (!ctx || !c) return SAI_ERR_NULL;
  if (layer < 0 || layer >= c->desc.num_layers)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "kv_cache_set_layer_window: layer_idx %d", layer);
  if (window < 0)
    return fail(ctx, SAI_ERR_INVALID_ATTRIBUTE, "kv_cache_set_layer_window: window %d < 0",
                window);
  c->layer_window[layer] = window;
  return SAI_OK;
}

SAI_API void sai_kvcache_destroy(sai_kvcache* c) {
  if (!c) return;
  for (uint8_t* p : c->pools)
    if (p) (void)hipFree(p);
  if (c->d_page_table) (void)hipFree(c->d_page_table);
  if (c->d_seq_lens) (void)hipFree(c->d_seq_lens);
  release_workspace(c->ws);
  delete c;
}

SAI_API sai_status sai_kvcache_set_page_table(sai_ctx* ctx, sai_kvcache* c,
                                              const int32_t* page_table, int32_t batch) {
  if (!ctx || !c || !page_table) return SAI_ERR_NULL;
  const sai_kvcache_desc& d = c->desc;
  if (batch <= 0 || batch > d.max_batch)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "set_page_table: batch %d not in 1..%d", batch,
                d.max_batch);
  const int w = d.max_pages_per_seq;
  std::vector<int32_t> mapped(d.max_batch, 0);
  for (int b = 0; b < batch; ++b) {
    int lead = 0;
    bool gap = false;
    for (int i = 0; i < w; ++i) {
      const int32_t pid = page_table[(size_t)b * w + i];
      if (pid < -1 || pid >= d.num_pages)
        return fail(ctx, SAI_ERR_SHAPE_MISMATCH,
                    "set_page_table: page id %d of sequence %d slot %d outside [0, %d)", pid, b, i,
                    d.num_pages);
      if (pid == -1) gap = true;
      if (!gap) lead = i + 1;
    }
    mapped[b] = lead;
  }
  DeviceGuard dg(ctx->device);
  // setup call: order after all work that may still read the table
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(ctx, e, "set_page_table: sync");
  std::vector<int32_t> dev_copy((size_t)batch * w);
  for (size_t i = 0; i < dev_copy.size(); ++i) dev_copy[i] = std::max(page_table[i], 0);
  e = hipMemcpy(c->d_page_table, dev_copy.data(), dev_copy.size() * sizeof(int32_t),
                hipMemcpyHostToDevice);
  if (e != hipSuccess) return hip_fail(ctx, e, "set_page_table");
  std::fill(c->h_page_table.begin(), c->h_page_table.end(), -1);
  std::copy(page_table, page_table + (size_t)batch * w, c->h_page_table.begin());
  c->h_mapped = mapped;
  c->batch = batch;
  std::fill(c->h_seq_lens.begin(), c->h_seq_lens.end(), 0);
  c->pending = 0;
  e = hipMemset(c->d_seq_lens, 0, (size_t)d.max_batch * sizeof(int32_t));
  if (e != hipSuccess) return hip_fail(ctx, e, "set_page_table: lengths");
  return SAI_OK;
}

SAI_API sai_status sai_kvcache_set_seq_lens(sai_ctx* ctx, sai_kvcache* c, const int32_t* seq_lens,
                                            int32_t batch) {
  if (!ctx || !c || !seq_lens) return SAI_ERR_NULL;
  if (batch != c->batch)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "set_seq_lens: batch %d != page table batch %d",
                batch, c->batch);
  for (int b = 0; b < batch; ++b) {
    if (seq_lens[b] < 0 || (int64_t)seq_lens[b] > (int64_t)c->h_mapped[b] * SAI_PAGE_TOKENS)
      return fail(ctx, SAI_ERR_OVERFLOW, "set_seq_lens: length %d of sequence %d exceeds %d mapped pages",
                  seq_lens[b], b, c->h_mapped[b]);
  }
  DeviceGuard dg(ctx->device);
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(ctx, e, "set_seq_lens: sync");
  e = hipMemcpy(c->d_seq_lens, seq_lens, (size_t)batch * sizeof(int32_t),
                           hipMemcpyHostToDevice);
  if (e != hipSuccess) return hip_fail(ctx, e, "set_seq_lens");
  std::copy(seq_lens, seq_lens + batch, c->h_seq_lens.begin());
  c->pending = 0;
  return SAI_OK;
}

SAI_API sai_status sai_kvcache_advance(sai_ctx* ctx, sai_kvcache* c, void* stream) {
  if (!ctx || !c) return SAI_ERR_NULL;
  if (c->pending == 0) return SAI_OK;
  for (int b = 0; b < c->batch; ++b)
    if ((int64_t)c->h_seq_lens[b] + c->pending > (int64_t)c->desc.max_pages_per_seq * SAI_PAGE_TOKENS)
      return fail(ctx, SAI_ERR_OVERFLOW, "kv_cache_advance:position_overflow");
  DeviceGuard dg(ctx->device);
  hipError_t e = sai::launch_seq_advance(c->d_seq_lens, c->batch, c->pending, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "kv_cache_advance");
  for (int b = 0; b < c->batch; ++b) c->h_seq_lens[b] += c->pending;
  c->pending = 0;
  return SAI_OK;
}

SAI_API sai_status sai_kvcache_reset(sai_ctx* ctx, sai_kvcache* c) {
  if (!ctx || !c) return SAI_ERR_NULL;
  DeviceGuard dg(ctx->device);
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemset(c->d_seq_lens, 0, (size_t)c->desc.max_batch * sizeof(int32_t));
  if (e != hipSuccess) return hip_fail(ctx, e, "kv_cache_reset");
  std::fill(c->h_seq_lens.begin(), c->h_seq_lens.end(), 0);
  c->pending = 0;
  return SAI_OK;
}

SAI_API sai_status sai_kvcache_lengths(const sai_kvcache* c, int32_t* seq_lens_out,
                                       int32_t* pending_out, int32_t* batch_out) {
  if (!c) return SAI_ERR_NULL;
  if (seq_lens_out) std::copy(c->h_seq_lens.begin(), c->h_seq_lens.begin() + c->batch, seq_lens_out);
  if (pending_out) *pending_out = c->pending;
  if (batch_out) *batch_out = c->batch;
  return SAI_OK;
}

SAI_API sai_status sai_kvcache_pool(const sai_kvcache* c, int32_t layer, void** dev_ptr,
                                    size_t* bytes, size_t* block_bytes) {
  if (!c) return SAI_ERR_NULL;
  if (layer < 0 || layer >= c->desc.num_layers) return SAI_ERR_SHAPE_MISMATCH;
  if (dev_ptr) *dev_ptr = c->pools[layer];
  if (bytes) *bytes = c->pool_bytes;
  if (block_bytes) *block_bytes = c->block_bytes;
  return SAI_OK;
}

SAI_API sai_status sai_kvcache_read(sai_ctx* ctx, sai_kvcache* c, int32_t layer, int32_t b,
                                    int32_t kv_head, int32_t t0, int32_t n_tokens, void* k_codes,
                                    void* v_codes, void* k_params, void* v_params) {
  if (!ctx || !c) return SAI_ERR_NULL;
  const sai_kvcache_desc& d = c->desc;
  if (layer < 0 || layer >= d.num_layers || b < 0 || b >= c->batch || kv_head < 0 ||
      kv_head >= d.num_kv_heads || t0 < 0 || n_tokens < 0)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "kvcache_read: index out of range");
  if ((int64_t)t0 + n_tokens > (int64_t)c->h_mapped[b] * SAI_PAGE_TOKENS)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "kvcache_read: tokens beyond the mapped pages");
  DeviceGuard dg(ctx->device);
  {
    // synchronous: the tokens of every append already enqueued on any stream
    const hipError_t es = hipDeviceSynchronize();
    if (es != hipSuccess) return hip_fail(ctx, es, "kvcache_read");
  }
  const int D = d.head_dim;
  const int DS = sai::stored_head_dim(D);  // the block's row width
  std::vector<uint8_t> blk(c->block_bytes);
  const int NG = D / 32;
  for (int t = t0; t < t0 + n_tokens; ++t) {
    const int page = c->h_page_table[(size_t)b * d.max_pages_per_seq + t / SAI_PAGE_TOKENS];
    const int slot = t % SAI_PAGE_TOKENS;
    const int i = t - t0;
    // one block copy per page (re-used while t stays in the page)
    if (i == 0 || slot == 0) {
      hipError_t e = hipMemcpy(blk.data(),
                               c->pools[layer] + sai::block_offset(page, kv_head, d.num_pages, c->block_bytes),
                               c->block_bytes, hipMemcpyDeviceToHost);
      if (e != hipSuccess) return hip_fail(ctx, e, "kvcache_read");
    }
    if (d.quant == SAI_KV_INT8) {
      // stored dim e -> the caller's dim (padding dims of the width 192 skipped)
      for (int e = 0; e < DS; ++e) {
        const int el = DS == D ? e : sai::logical_dim<192>(e);
        if (el < 0) continue;
        if (k_codes) ((int8_t*)k_codes)[(size_t)i * D + el] = (int8_t)blk[(size_t)slot * DS + e];
        if (v_codes) ((int8_t*)v_codes)[(size_t)i * D + el] = (int8_t)blk[16 * DS + e * 16 + slot];
      }
      if (k_params) std::memcpy((float*)k_params + i, blk.data() + 32 * DS + 4 * slot, 4);
      if (v_params) std::memcpy((float*)v_params + i, blk.data() + 32 * DS + 64 + 4 * slot, 4);
    } else {
      if (k_codes) std::memcpy((uint8_t*)k_codes + (size_t)i * (D / 2), blk.data() + (size_t)slot * (D / 2), D / 2);
      if (v_codes) {
        uint8_t* dst = (uint8_t*)v_codes + (size_t)i * (D / 2);
        for (int e = 0; e < D; e += 2) {
          const uint8_t b0 = blk[8 * D + e * 8 + slot / 2];
          const uint8_t b1 = blk[8 * D + (e + 1) * 8 + slot / 2];
          const uint8_t n0 = (slot & 1) ? (b0 >> 4) : (b0 & 0xF);
          const uint8_t n1 = (slot & 1) ? (b1 >> 4) : (b1 & 0xF);
          dst[e / 2] = (uint8_t)(n0 | (n1 << 4));
        }
      }
      if (k_params)
        std::memcpy((uint16_t*)k_params + (size_t)i * NG * 2, blk.data() + 16 * D + (size_t)slot * NG * 4, NG * 4);
      if (v_params)
        std::memcpy((uint16_t*)v_params + (size_t)i * NG * 2,
                    blk.data() + 16 * D + 64 * NG + (size_t)slot * NG * 4, NG * 4);
    }
  }
  return SAI_OK;
}

// ---------------------------------------------------------------- kernels ---
SAI_API sai_status sai_kv_append(sai_ctx* ctx, sai_kvcache* c, int32_t layer, const void* k,
                                 const void* v, int32_t dtype, int32_t batch, int32_t s_new,
                                 const float* cos_cache, const float* sin_cache, int32_t cache_rows,
                                 int32_t do_rotary, int32_t rotary_interleaved, void* stream) {
  if (!ctx || !c) return SAI_ERR_NULL;
  const char* op = "kv_append";
  if (!k || !v) return fail(ctx, SAI_ERR_NULL, "%s: missing key/value", op);
  if (layer < 0 || layer >= c->desc.num_layers)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "kv_cache_append:layer_idx %d", layer);
  if (dtype != SAI_DTYPE_F32 && dtype != SAI_DTYPE_BF16)
    return fail(ctx, SAI_ERR_UNSUPPORTED, "%s: dtype %d (want f32 or bf16)", op, dtype);
  if (s_new <= 0) return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "%s: s_new must be > 0", op);
  if (c->pending != 0 && c->pending != s_new)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH,
                "%s: %d tokens pending from another layer of this pass, got %d", op, c->pending,
                s_new);
  sai_status st = check_lengths(ctx, c, batch, s_new, op);
  if (st != SAI_OK) return st;
  st = check_rope(ctx, c, batch, s_new, cos_cache, sin_cache, cache_rows, do_rotary, op);
  if (st != SAI_OK) return st;
  DeviceGuard dg(ctx->device);
  sai::AppendParams p{};
  p.k = k;
  p.v = v;
  p.dtype = dtype;
  p.batch = batch;
  p.s_new = s_new;
  p.kv_heads = c->desc.num_kv_heads;
  p.cos_cache = cos_cache;
  p.sin_cache = sin_cache;
  p.cache_rows = cache_rows;
  p.do_rotary = do_rotary ? 1 : 0;
  p.interleaved = rotary_interleaved ? 1 : 0;
  p.seq_lens = c->d_seq_lens;
  p.page_table = c->d_page_table;
  p.max_pages = c->desc.max_pages_per_seq;
  p.pool = c->pools[layer];
  p.num_pages = c->desc.num_pages;
  // pages the new rows span, from the committed lengths (h_seq_lens mirrors
  // the device's)
  int32_t pages = 0;
  for (int b = 0; b < batch; ++b)
    pages = std::max(pages, (c->h_seq_lens[b] % SAI_PAGE_TOKENS + s_new + SAI_PAGE_TOKENS - 1) /
                                SAI_PAGE_TOKENS);
  p.pages = pages;
  hipError_t e = sai::launch_kv_append(p, c->desc.head_dim, c->desc.quant, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "kv_append launch");
  c->pending = s_new;
  return SAI_OK;
}

namespace {

sai_status attention_common(sai_ctx* ctx, sai_kvcache* c, int32_t layer, const void* q,
                            int32_t dtype, int32_t batch, int32_t sq, int32_t num_heads,
                            const float* cos_cache, const float* sin_cache, int32_t cache_rows,
                            int32_t do_rotary, const void* out, int32_t out_dtype,
                            const char* op, int32_t* group) {
  if (!q || !out) return fail(ctx, SAI_ERR_NULL, "%s: missing query/output", op);
  if (out_dtype != SAI_DTYPE_F32 && out_dtype != SAI_DTYPE_BF16)
    return fail(ctx, SAI_ERR_UNSUPPORTED, "%s: output dtype %d (want f32 or bf16)", op, out_dtype);
  if (layer < 0 || layer >= c->desc.num_layers)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "%s: layer_idx %d", op, layer);
  if (dtype != SAI_DTYPE_F32 && dtype != SAI_DTYPE_BF16)
    return fail(ctx, SAI_ERR_UNSUPPORTED, "%s: dtype %d (want f32 or bf16)", op, dtype);
  const int kvh = c->desc.num_kv_heads;
  if (num_heads <= 0)
    return fail(ctx, SAI_ERR_INVALID_ATTRIBUTE, "GroupQueryAttention: num_heads and kv_num_heads must be > 0");
  if (num_heads % kvh != 0)
    return fail(ctx, SAI_ERR_INVALID_ATTRIBUTE,
                "GroupQueryAttention: num_heads must be a multiple of kv_num_heads");
  const int G = num_heads / kvh;
  if (G != 1 && G != 2 && G != 4 && G != 8)
    return fail(ctx, SAI_ERR_UNSUPPORTED, "%s: group size %d (supported 1, 2, 4, 8)", op, G);
  if (c->pending != sq)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH,
                "%s: %d query tokens but %d tokens pending in the cache (append first)", op, sq,
                c->pending);
  sai_status st = check_lengths(ctx, c, batch, sq, op);
  if (st != SAI_OK) return st;
  st = check_rope(ctx, c, batch, sq, cos_cache, sin_cache, cache_rows, do_rotary, op);
  if (st != SAI_OK) return st;
  *group = G;
  return SAI_OK;
}

}  // namespace

namespace {

// Shared by sai_gqa_decode and sai_gqa_with_cache (k_new/v_new non-null: the
// decode kernel appends the step's token itself).
sai_status launch_decode(sai_ctx* ctx, sai_kvcache* c, int32_t layer, const void* q,
                         int32_t dtype, int32_t batch, int32_t G, const float* cos_cache,
                         const float* sin_cache, int32_t cache_rows, int32_t do_rotary,
                         int32_t rotary_interleaved, int32_t has_scale, float scale,
                         int32_t window, void* out, int32_t out_dtype, const void* k_new,
                         const void* v_new, int32_t kv_dtype, void* stream,
                         DecodeWorkspace* fixed_ws = nullptr) {
  const char* op = "gqa_decode";
  const int32_t W = visible_span(c->layer_window[layer], window);
  const int D = c->desc.head_dim;
  if (D == 256 && G > 4 && c->desc.quant == SAI_KV_INT4)
    return fail(ctx, SAI_ERR_UNSUPPORTED,
                "%s: int4 at head_dim 256 supports groups of 1, 2 and 4 (got %d)",
                op, G);
  const int kvh = c->desc.num_kv_heads;

  // Split size. Uniform lengths: one round of about one workgroup per CU
  // (each streams one contiguous range; measured best at 16 x 8k). Ragged
  // lengths: cap the split so the longest sequences are cut into pieces that
  // balance across the CUs (64 x U[128, 16384] tokens, 8 kv heads: 181.4 us
  // per step at 3072, 182.3 at 2560, 183.6 at 2816, 185.1 at 2048, 185.4 at
  // 3584, 188.3 at 4096).
  // streamed tokens of sequence b: from the tile of its first visible key
  auto streamed = [&](int b) {
    const int L = c->h_seq_lens[b] + 1;
    return (int64_t)(L - sai::window_origin(L, W));
  };
  int64_t tok_heads = 0;
  int64_t max_len = 0;
  for (int b = 0; b < batch; ++b) {
    tok_heads += streamed(b) * kvh;
    max_len = std::max<int64_t>(max_len, streamed(b));
  }
  int32_t split = ctx->decode_split;
  if (split <= 0) {
    int64_t s = (tok_heads + ctx->num_cus - 1) / ctx->num_cus;
    const int64_t mean_len = std::max<int64_t>(1, tok_heads / ((int64_t)kvh * batch));
    if (max_len > 2 * mean_len) s = std::min<int64_t>(s, 3072);
    s = ((s + 63) / 64) * 64;
    split = (int32_t)std::max<int64_t>(256, std::min<int64_t>(s, kMaxDecodeSplit));
    // At the 256-token floor each wave streams one tile. A batch whose
    // sequences all fit one 512-token split takes one split each (no merge, no
    // short remainder split): 1 x 512 tokens (8Q/2KV, head_dim 64) 7.83 ->
    // 7.68 us per step, 16 x 300 (32Q/8KV, 128) 11.66 -> 10.95 us. Sequences
    // cut into more than 8 such splits take 512 too: 1 x 8192 (32Q/8KV)
    // 18.5 -> 14.7 us, 2 x 3000 13.8 -> 13.3, 1 x 16384 (8Q/1KV) 38.8 ->
    // 29.9. Between the two, 256 stays (4 x 1000: 11.5 against 12.9 us).
    // The int4 kernel's 8-wave workgroups measured the other way at 16 x 300
    // (11.0 us at 256 against 11.3) and 2 x 3000 (12.5 against 13.2, twelve
    // splits), so int4 takes 512 only past 16 splits (1 x 8192: 14.5 -> 13.7).
    const int64_t splits256 = (max_len + 255) / 256;
    if (split < 512 && (c->desc.quant == SAI_KV_INT8 ? (max_len <= 512 || splits256 > 8)
                                                     : splits256 > 16))
      split = 512;
  }
  split = std::min(split, kMaxDecodeSplit);
  int64_t work = 0;
  bool multi = false;
  int64_t n_first = -1, n_max = 0;
  bool uniform = true;
  for (int b = 0; b < batch; ++b) {
    const int64_t n = (streamed(b) + split - 1) / split;
    work += n;
    multi = multi || n > 1;
    if (n_first < 0) n_first = n;
    uniform = uniform && n == n_first;
    n_max = std::max(n_max, n);
  }
  if (work <= 0 || work > 0x7FFFFFFF)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "%s: bad work size", op);
  DeviceGuard dg(ctx->device);
  // the cache's own workspace (sized at creation for the automatic split; a
  // smaller split set for tuning may grow it once, synchronously), or a fixed
  // one that cannot grow
  const size_t need_partials = (size_t)work * kvh * G * (sai::stored_head_dim(D) + 2);
  DecodeWorkspace* ws = &c->ws;
  if (fixed_ws) {
    if (need_partials > fixed_ws->partial_floats || (size_t)batch * 2 > fixed_ws->seq_info_n ||
        (size_t)batch * kvh > fixed_ws->counter_n)
      return fail(ctx, SAI_ERR_UNSUPPORTED,
                  "%s: the step needs %zu partial floats, %d sequences and %d (sequence, kv head) "
                  "pairs; the fixed scratch holds %zu, %zu and %zu",
                  op, need_partials, batch, batch * kvh, fixed_ws->partial_floats,
                  fixed_ws->seq_info_n / 2, fixed_ws->counter_n);
    ws = fixed_ws;
  } else {
    sai_status st = reserve_workspace(ctx, c->ws, need_partials, (size_t)batch * 2,
                                      (size_t)batch * kvh);
    if (st != SAI_OK) return st;
  }

  sai::DecodeParams p{};
  p.q = q;
  p.q_dtype = dtype;
  p.out = out;
  p.out_bf16 = out_dtype == SAI_DTYPE_BF16 ? 1 : 0;
  p.pool = c->pools[layer];
  p.kv_heads = kvh;
  p.num_pages = c->desc.num_pages;
  p.seq_lens = c->d_seq_lens;
  p.pending = 1;
  p.page_table = c->d_page_table;
  p.max_pages = c->desc.max_pages_per_seq;
  p.batch = batch;
  p.cos_cache = cos_cache;
  p.sin_cache = sin_cache;
  p.cache_rows = cache_rows;
  p.do_rotary = do_rotary ? 1 : 0;
  p.interleaved = rotary_interleaved ? 1 : 0;
  const float sc = has_scale ? scale : sai_default_scale(D);
  p.scale_log2 = sc * 1.4426950408889634f;
  p.split_tokens = split;
  // int4 tiles are compute-heavier: two waves per SIMD from one workgroup
  p.waves = ctx->decode_waves ? ctx->decode_waves : (c->desc.quant == SAI_KV_INT4 ? 8 : 4);
  p.uniform_nsplit = uniform ? (int)n_first : 0;
  p.max_nsplit = (int)n_max;
  p.partials = ws->partials;
  p.seq_info = ws->seq_info;
  // automatic: the last workgroup merges when every sequence has the same
  // split count (one ticket per (sequence, kv head), measured faster at 16 x
  // 8k, int8, and at 4 x 32k, int4); ragged batches use the combine kernel
  // (measured faster there).
  p.merge_in_kernel = ctx->decode_merge == 1 || (ctx->decode_merge == 2 && uniform);
  p.static_tiles = ctx->reproducible != 0;
  // ragged: work items go to the sequences with the longest splits first
  // (each sequence's tiles are dealt evenly to its splits, so this orders the
  // work items longest first), which the in-order dispatch of workgroups to
  // CUs then balances as a longest-processing-time list schedule
  p.ordered = 0;
  if (!uniform && batch <= sai::kDecodeOrder) {
    std::vector<std::pair<int64_t, int>> key((size_t)batch);
    for (int b = 0; b < batch; ++b) {
      const int64_t tiles = (streamed(b) + 63) / 64;
      const int64_t n = (streamed(b) + split - 1) / split;
      key[b] = {-((tiles + n - 1) / n), b};
    }
    std::stable_sort(key.begin(), key.end());
    for (int i = 0; i < batch; ++i) p.order[i] = (uint16_t)key[i].second;
    p.ordered = 1;
  }
  p.counters = ws->counters;
  p.k_new = k_new;
  p.v_new = v_new;
  p.kv_dtype = kv_dtype;
  p.window = W;
  const hipStream_t hs = (hipStream_t)stream;
  const int64_t slots = (int64_t)ctx->ev_start.size();
  const int64_t slot = slots ? ctx->timed_calls % slots : 0;
  if (slots) {
    const hipError_t ee = hipEventRecord(ctx->ev_start[slot], hs);
    if (ee != hipSuccess) return hip_fail(ctx, ee, "gqa_decode timing event");
  }
  // the decode kernel, then (several splits, merge not in-kernel) the combine
  hipError_t e = sai::launch_gqa_decode(p, D, G, c->desc.quant, (int)work, false, hs);
  if (e != hipSuccess) return hip_fail(ctx, e, "gqa_decode launch");
  if (slots) {
    e = hipEventRecord(ctx->ev_end[slot], hs);
    if (e != hipSuccess) return hip_fail(ctx, e, "gqa_decode timing event");
    ++ctx->timed_calls;
  }
  if (multi && !p.merge_in_kernel) {
    e = sai::launch_decode_combine(p, D, G, hs);
    if (e != hipSuccess) return hip_fail(ctx, e, "gqa_decode combine launch");
  }
  ctx->last_wg = (int32_t)(work * kvh);
  ctx->last_split = split;
  ctx->last_launches = (multi && !p.merge_in_kernel) ? 2 : 1;
  return SAI_OK;
}

}  // namespace

SAI_API sai_status sai_gqa_decode(sai_ctx* ctx, sai_kvcache* c, int32_t layer, const void* q,
                                  int32_t dtype, int32_t batch, int32_t num_heads,
                                  const float* cos_cache, const float* sin_cache,
                                  int32_t cache_rows, int32_t do_rotary,
                                  int32_t rotary_interleaved, int32_t has_scale, float scale,
                                  int32_t window, void* out, int32_t out_dtype, void* stream) {
  if (!ctx || !c) return SAI_ERR_NULL;
  int32_t G = 0;
  sai_status st = attention_common(ctx, c, layer, q, dtype, batch, 1, num_heads, cos_cache,
                                   sin_cache, cache_rows, do_rotary, out, out_dtype, "gqa_decode",
                                   &G);
  if (st != SAI_OK) return st;
  return launch_decode(ctx, c, layer, q, dtype, batch, G, cos_cache, sin_cache, cache_rows,
                       do_rotary, rotary_interleaved, has_scale, scale, window, out, out_dtype,
                       nullptr, nullptr, SAI_DTYPE_F32, stream);
}

namespace {

sai_status gqa_with_cache_impl(sai_ctx* ctx, sai_kvcache* c, int32_t layer, const void* q,
                               int32_t q_dtype, const void* k_new, const void* v_new,
                               int32_t kv_dtype, int32_t batch, int32_t num_heads,
                               const float* cos_cache, const float* sin_cache,
                               int32_t cache_rows, int32_t do_rotary, int32_t rotary_interleaved,
                               int32_t has_scale, float scale, int32_t window, void* out,
                               int32_t out_dtype, void* stream, const char* op,
                               DecodeWorkspace* fixed_ws) {
  if (!k_new || !v_new) return fail(ctx, SAI_ERR_NULL, "%s: missing key/value", op);
  if (kv_dtype != SAI_DTYPE_F32 && kv_dtype != SAI_DTYPE_BF16)
    return fail(ctx, SAI_ERR_UNSUPPORTED, "%s: dtype %d (want f32 or bf16)", op, kv_dtype);
  if (c->pending != 0 && c->pending != 1)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH,
                "%s: %d tokens pending from another layer of this pass, got 1", op, c->pending);
  // the token appended here is the pending one the attention sees
  const int32_t prev_pending = c->pending;
  c->pending = 1;
  int32_t G = 0;
  sai_status st = attention_common(ctx, c, layer, q, q_dtype, batch, 1, num_heads, cos_cache,
                                   sin_cache, cache_rows, do_rotary, out, out_dtype, op, &G);
  if (st == SAI_OK)
    st = launch_decode(ctx, c, layer, q, q_dtype, batch, G, cos_cache, sin_cache, cache_rows,
                       do_rotary, rotary_interleaved, has_scale, scale, window, out, out_dtype,
                       k_new, v_new, kv_dtype, stream, fixed_ws);
  if (st != SAI_OK) c->pending = prev_pending;
  return st;
}

}  // namespace

SAI_API sai_status sai_gqa_with_cache(sai_ctx* ctx, sai_kvcache* c, int32_t layer,
                                      const void* q, int32_t q_dtype, const void* k_new,
                                      const void* v_new, int32_t kv_dtype, int32_t batch,
                                      int32_t num_heads, const float* cos_cache,
                                      const float* sin_cache, int32_t cache_rows,
                                      int32_t do_rotary, int32_t rotary_interleaved,
                                      int32_t has_scale, float scale, int32_t window, void* out,
                                      int32_t out_dtype, void* stream) {
  if (!ctx || !c) return SAI_ERR_NULL;
  return gqa_with_cache_impl(ctx, c, layer, q, q_dtype, k_new, v_new, kv_dtype, batch, num_heads,
                             cos_cache, sin_cache, cache_rows, do_rotary, rotary_interleaved,
                             has_scale, scale, window, out, out_dtype, stream, "gqa_with_cache",
                             nullptr);
}

SAI_API sai_status sai_gqa_with_cache_noalloc(sai_ctx* ctx, sai_kvcache* c, int32_t layer,
                                              const void* q, int32_t q_dtype, const void* k_new,
                                              const void* v_new, int32_t kv_dtype, int32_t batch,
                                              int32_t num_heads, const float* cos_cache,
                                              const float* sin_cache, int32_t cache_rows,
                                              int32_t do_rotary, int32_t rotary_interleaved,
                                              int32_t has_scale, float scale, int32_t window,
                                              void* out, int32_t out_dtype, void* stream) {
  if (!ctx || !c) return SAI_ERR_NULL;
  const char* op = "gqa_with_cache_noalloc";
  void* base = nullptr;
  if (ctx->device < kMaxScratchDevices) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    base = g_scratch[ctx->device].ptr;
  }
  if (!base)
    return fail(ctx, SAI_ERR_HIP, "%s: the device scratch of device %d is not set up", op,
                ctx->device);
  // counters, then split ranges, then partials. Every launch that merges
  // in-kernel leaves its counters at zero; they are cleared again on the
  // caller's stream before each call anyway, so that what an overlapping
  // (racing) call left behind cannot reach a later one.
  DecodeWorkspace ws;
  ws.counters = (int32_t*)base;
  ws.counter_n = kScratchCounters;
  ws.seq_info = (int32_t*)base + kScratchCounters;
  ws.seq_info_n = kScratchSeqInfo;
  ws.partials = (float*)((int32_t*)base + kScratchCounters + kScratchSeqInfo);
  ws.partial_floats = kScratchPartialFloats;
  if (batch > 0 && (size_t)batch * c->desc.num_kv_heads <= kScratchCounters) {
    DeviceGuard dg(ctx->device);
    const hipError_t e = sai::launch_fill_i32(ws.counters, (size_t)batch * c->desc.num_kv_heads,
                                              0, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "gqa_with_cache_noalloc: counter clear");
  }
  return gqa_with_cache_impl(ctx, c, layer, q, q_dtype, k_new, v_new, kv_dtype, batch, num_heads,
                             cos_cache, sin_cache, cache_rows, do_rotary, rotary_interleaved,
                             has_scale, scale, window, out, out_dtype, stream, op, &ws);
}

SAI_API sai_status sai_gqa_prefill(sai_ctx* ctx, sai_kvcache* c, int32_t layer, const void* q,
                                   int32_t dtype, int32_t batch, int32_t sq, int32_t num_heads,
                                   const float* cos_cache, const float* sin_cache,
                                   int32_t cache_rows, int32_t do_rotary,
                                   int32_t rotary_interleaved, int32_t has_scale, float scale,
                                   int32_t window, void* out, int32_t out_dtype, void* stream) {
  if (!ctx || !c) return SAI_ERR_NULL;
  const char* op = "gqa_prefill";
  if (sq <= 0) return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "%s: sq must be > 0", op);
  int32_t G = 0;
  sai_status st = attention_common(ctx, c, layer, q, dtype, batch, sq, num_heads, cos_cache,
                                   sin_cache, cache_rows, do_rotary, out, out_dtype, op, &G);
  if (st != SAI_OK) return st;
  const int D = c->desc.head_dim;
  DeviceGuard dg(ctx->device);
  sai::PrefillParams p{};
  p.q = q;
  p.q_dtype = dtype;
  p.out = out;
  p.out_bf16 = out_dtype == SAI_DTYPE_BF16 ? 1 : 0;
  p.pool = c->pools[layer];
  p.kv_heads = c->desc.num_kv_heads;
  p.num_pages = c->desc.num_pages;
  p.seq_lens = c->d_seq_lens;
  p.sq = sq;
  p.page_table = c->d_page_table;
  p.max_pages = c->desc.max_pages_per_seq;
  p.batch = batch;
  p.cos_cache = cos_cache;
  p.sin_cache = sin_cache;
  p.cache_rows = cache_rows;
  p.do_rotary = do_rotary ? 1 : 0;
  p.interleaved = rotary_interleaved ? 1 : 0;
  const float sc = has_scale ? scale : sai_default_scale(D);
  p.scale_log2 = sc * 1.4426950408889634f;
  p.window = visible_span(c->layer_window[layer], window);
  // Key split: a short chunk over a long past has few workgroups (one per
  // 256 rows and kv head), each streaming the whole visible past. With fewer
  // than 256 of them (one per CU) and at least 16 tiles to stream, the rows'
  // key range is cut into splits of at least 4 tiles, to about 256
  // workgroups, and the decode's combine kernel merges the partials (each row
  // of the chunk a sequence of its own). 1 x 8192 past, 32Q/8KV: 16 tokens
  // 334 -> 35 us, 1024 tokens 381 -> 228 us (the c5 chunk has 512 workgroups).
  int64_t max_past = 0;
  for (int b = 0; b < batch; ++b) max_past = std::max<int64_t>(max_past, c->h_seq_lens[b]);
  const int64_t key_tiles = (max_past + sq + 63) / 64;
  const int64_t base_wgs = (int64_t)sai::prefill_workgroups(p, D, G);
  int nks = 1;
  if (base_wgs < 256 && key_tiles >= 16)
    nks = (int)std::min<int64_t>((256 + base_wgs - 1) / base_wgs, key_tiles / 4);
  if (nks > 1) {
    p.nksplit = nks;
    p.ksplit_tiles = (int)((key_tiles + nks - 1) / nks);
    const size_t rows = (size_t)batch * sq;
    const size_t need =
        rows * nks * c->desc.num_kv_heads * G * (size_t)(sai::stored_head_dim(D) + 2);
    st = reserve_workspace(ctx, c->ws, need, 0, 0);
    if (st != SAI_OK) return st;
    p.partials = c->ws.partials;
  }
  st = reserve_prec_flags(ctx, c->ws, sai::prefill_workgroups(p, D, G));
  if (st != SAI_OK) return st;
  p.prec_flags = c->ws.prec_flags;
  hipError_t e = sai::launch_gqa_prefill(p, D, G, c->desc.quant, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "gqa_prefill launch");
  if (nks > 1) {
    sai::DecodeParams m{};
    m.out = out;
    m.out_bf16 = p.out_bf16;
    m.kv_heads = c->desc.num_kv_heads;
    m.batch = batch * sq;
    m.uniform_nsplit = nks;
    m.max_nsplit = nks;
    m.partials = c->ws.partials;
    e = sai::launch_decode_combine(m, D, G, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "gqa_prefill key-split merge");
  }
  return SAI_OK;
}

// ------------------------------------------------ standalone rotary embedding ---
namespace {

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Launches over sequences [b0, b0 + nb) x sequence indices [s0, s0 + ns) with
// the positions `tab` (mode 0: one start per sequence, mode 1: one position
// per sequence index). Splits the range so that every launch holds at most
// sai::kRotaryTab positions and fewer than 2^31 work items.
struct RotaryPlan {
  sai::RotaryArgs base;
  bool x_bf16, t_bf16, interleaved;
  hipStream_t st;
  uint64_t unit;  // work items of one (b, s) step: head_groups * items
};

constexpr uint64_t kRotaryMaxItems = (uint64_t)1 << 31;

hipError_t rotary_launch_range(const RotaryPlan& pl, int mode, int32_t b0, int32_t nb,
                               int32_t s0, int32_t ns, const int32_t* tab) {
  sai::RotaryArgs a = pl.base;
  a.mode = mode;
  a.b0 = b0;
  a.s0 = s0;
  a.ns = ns;
  const uint64_t total = (uint64_t)nb * (uint64_t)ns * pl.unit;
  a.total = (uint32_t)total;
  const int n = mode == 0 ? nb : ns;
  for (int i = 0; i < n; ++i) a.tab[i] = tab[i];
  return sai::launch_rotary(a, pl.x_bf16, pl.t_bf16, pl.interleaved, pl.st);
}

// Mode 0 over all sequences: row position = start[b] + s.
hipError_t rotary_affine(const RotaryPlan& pl, int32_t batch, int32_t seq,
                         const std::vector<int32_t>& start) {
  const int32_t ns_max = (int32_t)std::min<uint64_t>((uint64_t)seq, kRotaryMaxItems / pl.unit);
  for (int32_t s0 = 0; s0 < seq; s0 += ns_max) {
    const int32_t ns = std::min(ns_max, seq - s0);
    const uint64_t per_b = (uint64_t)ns * pl.unit;
    const int32_t nb_max =
        (int32_t)std::min<uint64_t>((uint64_t)sai::kRotaryTab, kRotaryMaxItems / per_b);
    for (int32_t b0 = 0; b0 < batch; b0 += nb_max) {
      const int32_t nb = std::min(nb_max, batch - b0);
      hipError_t e = rotary_launch_range(pl, 0, b0, nb, s0, ns, start.data() + b0);
      if (e != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

// Mode 1 over sequences [b0, b0 + nb): row position = pos[s].
hipError_t rotary_explicit(const RotaryPlan& pl, int32_t b0, int32_t nb, int32_t seq,
                           const int32_t* pos) {
  const int32_t ns_max = (int32_t)std::min<uint64_t>(
      (uint64_t)sai::kRotaryTab, kRotaryMaxItems / pl.unit);
  for (int32_t s0 = 0; s0 < seq; s0 += ns_max) {
    const int32_t ns = std::min(ns_max, seq - s0);
    const int32_t nb_max = (int32_t)std::max<uint64_t>(
        1, std::min<uint64_t>((uint64_t)nb, kRotaryMaxItems / ((uint64_t)ns * pl.unit)));
    for (int32_t bb = 0; bb < nb; bb += nb_max) {
      const int32_t n = std::min(nb_max, nb - bb);
      hipError_t e = rotary_launch_range(pl, 1, b0 + bb, n, s0, ns, pos + s0);
      if (e != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

}  // namespace

SAI_API sai_status sai_rotary_embedding(sai_ctx* ctx, const void* x, void* y, int32_t dtype,
                                        int32_t batch, int32_t num_heads, int32_t seq,
                                        int32_t head_dim, int32_t layout,
                                        const int64_t* position_ids, int64_t n_pos,
                                        int64_t start_position, const void* cos_cache,
                                        const void* sin_cache, int32_t table_dtype,
                                        int32_t cache_rows, int32_t cache_cols, int32_t rotary_dim,
                                        int32_t interleaved, void* stream) {
  if (!ctx) return SAI_ERR_NULL;
  const char* op = "sai_rotary_embedding";
  if (dtype != SAI_DTYPE_F32 && dtype != SAI_DTYPE_BF16)
    return fail(ctx, SAI_ERR_UNSUPPORTED, "%s: dtype %d (need F32 or BF16)", op, dtype);
  if (table_dtype != SAI_DTYPE_F32 && table_dtype != SAI_DTYPE_BF16)
    return fail(ctx, SAI_ERR_UNSUPPORTED, "%s: table dtype %d (need F32 or BF16)", op,
                table_dtype);
  if (layout != SAI_ROPE_BHSD && layout != SAI_ROPE_BSHD)
    return fail(ctx, SAI_ERR_INVALID_ATTRIBUTE, "%s: unknown layout %d", op, layout);
  if (batch < 0 || num_heads < 0 || seq < 0 || head_dim < 0 || cache_rows < 0)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "%s: negative dimension", op);
  // apply_rope_in_place's order of checks (ops/microsoft.rs:197-232)
  const int64_t bs = (int64_t)batch * seq;
  if (position_ids && n_pos != bs && n_pos != seq)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH,
                "apply_rope_in_place: position_ids length %lld != B*Sq = %lld", (long long)n_pos,
                (long long)bs);
  if (!cos_cache || !sin_cache)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "RotaryEmbedding: missing %s",
                cos_cache ? "sin_cache" : "cos_cache");
  const int32_t rd = rotary_dim <= 0 ? head_dim : rotary_dim;
  if (rd == 0 || rd > head_dim)
    return fail(ctx, SAI_ERR_INVALID_ATTRIBUTE,
                "apply_rope_in_place: rotary_dim must be in 1..=head_dim");
  if (rd % 2 != 0)
    return fail(ctx, SAI_ERR_INVALID_ATTRIBUTE, "apply_rope_in_place: rotary_dim must be even");
  const int32_t half = rd / 2;
  if (cache_cols != half)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH,
                "apply_rope_in_place: cache inner dim %d != rotary_dim/2 = %d", cache_cols, half);
  const bool any_rows = batch > 0 && num_heads > 0 && seq > 0;
  // Positions: every row's table row is checked here, so the kernel reads
  // only rows that exist.
  std::vector<int32_t> start;  // per sequence, when every sequence is start + s
  std::vector<int32_t> pos;    // explicit, [n_pos]
  bool shared = false;
  if (position_ids) {
    shared = n_pos == seq;
    if (any_rows) {
      for (int32_t b = 0; b < batch; ++b)
        for (int32_t s = 0; s < seq; ++s) {
          const int64_t p = shared ? position_ids[s] : position_ids[(int64_t)b * seq + s];
          if (p < 0 || p >= cache_rows)
            return fail(ctx, SAI_ERR_SHAPE_MISMATCH,
                        "apply_rope_in_place: position %lld out of cache range %d", (long long)p,
                        cache_rows);
        }
      const int64_t n = shared ? seq : bs;
      pos.resize((size_t)n);
      for (int64_t i = 0; i < n; ++i) pos[(size_t)i] = (int32_t)position_ids[i];
      // one start per sequence when the ids run start, start + 1, ...
      bool affine = true;
      const int32_t nseq = shared ? 1 : batch;
      for (int32_t b = 0; b < nseq && affine; ++b)
        for (int32_t s = 1; s < seq; ++s)
          if (pos[(size_t)b * seq + s] != pos[(size_t)b * seq] + s) {
            affine = false;
            break;
          }
      if (affine) {
        start.resize((size_t)batch);
        for (int32_t b = 0; b < batch; ++b) start[(size_t)b] = pos[shared ? 0 : (size_t)b * seq];
      }
    }
  } else {
    // rotary_gpu (rotary.rs:247-252): the start and the whole run must be rows
    if (start_position < 0 || start_position + seq > cache_rows)
      return fail(ctx, SAI_ERR_SHAPE_MISMATCH,
                  "rotary_gpu: position + seq_len exceeds cos/sin table length (%lld + %d > %d)",
                  (long long)start_position, seq, cache_rows);
    start.assign((size_t)batch, (int32_t)start_position);
  }
  if (!any_rows) return SAI_OK;
  if (!x || !y) return fail(ctx, SAI_ERR_NULL, "%s: x or y is NULL", op);

  // vector path: 4 or 8 pairs per item with 8- to 64-byte accesses (every
  // row, half row and table row then starts on a multiple of the access);
  // the heads of an item share its cos/sin loads. bf16 rows: 8 pairs x 2
  // heads (16-byte row loads); f32 rows: 4 pairs x 4 heads.
  const bool vec = half % 4 == 0 && head_dim % 8 == 0 && aligned16(x) && aligned16(y) &&
                   aligned16(cos_cache) && aligned16(sin_cache);
  const int32_t P = !vec ? 1 : (dtype == SAI_DTYPE_BF16 && half % 8 == 0 ? 8 : 4);
  const int32_t NH = !vec ? 1 : (P == 8 ? 2 : 4);
  RotaryPlan pl{};
  pl.base.x = x;
  pl.base.y = y;
  pl.base.cos = cos_cache;
  pl.base.sin = sin_cache;
  pl.base.rot_items = half / P;
  pl.base.items = pl.base.rot_items + (x != y ? (head_dim - rd) / P : 0);
  pl.base.pairs_per_item = P;
  pl.base.heads_per_item = NH;
  pl.base.head_groups = (num_heads + NH - 1) / NH;
  pl.base.heads = num_heads;
  pl.base.seq = seq;
  pl.base.head_dim = head_dim;
  pl.base.rot_dim = rd;
  pl.base.cache_cols = cache_cols;
  pl.base.layout = layout;
  pl.x_bf16 = dtype == SAI_DTYPE_BF16;
  pl.t_bf16 = table_dtype == SAI_DTYPE_BF16;
  pl.interleaved = interleaved != 0;
  pl.st = (hipStream_t)stream;
  pl.unit = (uint64_t)pl.base.head_groups * (uint64_t)pl.base.items;
  if (pl.unit == 0) return SAI_OK;
  if (pl.unit >= kRotaryMaxItems)
    return fail(ctx, SAI_ERR_UNSUPPORTED, "%s: %d head groups x %d items per step exceed 2^31", op,
                pl.base.head_groups, pl.base.items);
  DeviceGuard dg(ctx->device);
  hipError_t e = hipSuccess;
  if (!start.empty()) {
    e = rotary_affine(pl, batch, seq, start);
  } else if (shared) {
    e = rotary_explicit(pl, 0, batch, seq, pos.data());
  } else {
    for (int32_t b = 0; b < batch && e == hipSuccess; ++b)
      e = rotary_explicit(pl, b, 1, seq, pos.data() + (size_t)b * seq);
  }
  if (e != hipSuccess) return hip_fail(ctx, e, "rotary launch");
  return SAI_OK;
}

SAI_API sai_status sai_rope_tables(sai_ctx* ctx, float rope_theta, int32_t max_pos, int32_t half,
                                   int32_t dtype, void* cos_out, void* sin_out, void* stream) {
  if (!ctx) return SAI_ERR_NULL;
  if (dtype != SAI_DTYPE_F32 && dtype != SAI_DTYPE_BF16)
    return fail(ctx, SAI_ERR_UNSUPPORTED, "sai_rope_tables: dtype %d (need BF16 or F32)", dtype);
  if (max_pos < 0 || half < 0)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "sai_rope_tables: negative size");
  const uint64_t n = (uint64_t)max_pos * (uint64_t)half;
  if (n >= kRotaryMaxItems)
    return fail(ctx, SAI_ERR_UNSUPPORTED, "sai_rope_tables: %d x %d entries exceed 2^31", max_pos,
                half);
  if (n == 0) return SAI_OK;
  if (!cos_out || !sin_out) return fail(ctx, SAI_ERR_NULL, "sai_rope_tables: NULL output");
  DeviceGuard dg(ctx->device);
  hipError_t e = sai::launch_rope_tables(rope_theta, (uint32_t)max_pos, (uint32_t)half,
                                         dtype == SAI_DTYPE_BF16, cos_out, sin_out,
                                         (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "rope_tables launch");
  return SAI_OK;
}

// ------------------------------------------------------------------ row copy ---
SAI_API sai_status sai_copy_rows(sai_ctx* ctx, const void* src, int32_t src_layout, void* dst,
                                 int32_t dst_layout, int32_t dtype, int32_t batch, int32_t heads,
                                 int32_t seq, int32_t head_dim, int32_t dst_seq,
                                 int32_t dst_offset, void* stream) {
  if (!ctx) return SAI_ERR_NULL;
  const char* op = "sai_copy_rows";
  if (dtype != SAI_DTYPE_F32 && dtype != SAI_DTYPE_BF16)
    return fail(ctx, SAI_ERR_UNSUPPORTED, "%s: dtype %d (need F32 or BF16)", op, dtype);
  if ((src_layout != SAI_ROPE_BHSD && src_layout != SAI_ROPE_BSHD) ||
      (dst_layout != SAI_ROPE_BHSD && dst_layout != SAI_ROPE_BSHD))
    return fail(ctx, SAI_ERR_INVALID_ATTRIBUTE, "%s: unknown layout", op);
  if (batch < 0 || heads < 0 || seq < 0 || head_dim < 0 || dst_offset < 0 ||
      (int64_t)dst_offset + seq > (int64_t)dst_seq)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH,
                "%s: rows [%d, %d + %d) do not fit a destination of %d positions", op, dst_offset,
                dst_offset, seq, dst_seq);
  const uint64_t rows = (uint64_t)batch * (uint64_t)heads * (uint64_t)seq;
  if (rows == 0 || head_dim == 0) return SAI_OK;
  if (!src || !dst) return fail(ctx, SAI_ERR_NULL, "%s: src or dst is NULL", op);
  const size_t esz = dtype == SAI_DTYPE_BF16 ? 2 : 4;
  const size_t row_bytes = (size_t)head_dim * esz;
  const int chunk = (row_bytes % 16 == 0 && aligned16(src) && aligned16(dst)) ? 16 : (int)esz;
  sai::CopyRowsArgs a{};
  a.src = src;
  a.dst = dst;
  a.chunks = (int32_t)(row_bytes / (size_t)chunk);
  a.total = rows * (uint64_t)a.chunks;
  a.heads = heads;
  a.seq = seq;
  a.dst_seq = dst_seq;
  a.dst_offset = dst_offset;
  a.src_layout = src_layout;
  a.dst_layout = dst_layout;
  DeviceGuard dg(ctx->device);
  const hipError_t e = sai::launch_copy_rows(a, chunk, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "copy_rows launch");
  return SAI_OK;
}

// ------------------------------------------------------- TurboQuant KV cache ---
namespace {

// sqrt_approx (onnx-rt/src/operators.rs:3311-3320), the WHT normalisation's
// square root: ten Newton steps from x, each op rounded on its own.
float sqrt_approx_newton(float x) {
  if (x <= 0.0f) return 0.0f;
  volatile float s = x;
  for (int i = 0; i < 10; ++i) {
    volatile float q = x / s;
    volatile float t = s + q;
    s = 0.5f * t;
  }
  return s;
}

// PolarQuantizer::new's signs (kv_compression.rs:197-214) from the cache's
// per-head seed (CompressedKVCache::new, :766-790).
void tq_rotation_signs(uint64_t seed, int layer, int heads, int head, int dim, int8_t* out) {
  const uint64_t head_seed = seed * 0x9E3779B97F4A7C15ull + (uint64_t)((int64_t)layer * heads + head);
  uint64_t st = head_seed ? head_seed : 0x5EEDDEADBEEFCAFEull;
  for (int i = 0; i < dim; ++i) {
    st ^= st << 13;
    st ^= st >> 7;
    st ^= st << 17;
    out[i] = (st & 1u) == 0 ? 1 : -1;
  }
}

sai::TqArgs tq_args(const sai_tqcache* c, int32_t layer) {
  const sai_tqcache::Layer& L = c->layers[layer];
  sai::TqArgs a{};
  a.codes_k = L.codes_k;
  a.codes_v = L.codes_v;
  a.par_k = L.par_k;
  a.par_v = L.par_v;
  a.signs_k = L.sg_k;
  a.signs_v = L.sg_v;
  a.signs = L.rot;
  a.seq_lens = c->d_lens;
  a.pending = c->pending;
  a.heads = c->desc.num_kv_heads;
  a.batch_cap = c->desc.max_batch;
  a.rows_cap = c->desc.max_rows;
  a.tiles_cap = c->tiles_cap;
  a.head_dim = c->desc.head_dim;
  a.bits = c->desc.bits;
  a.qjl = c->desc.qjl;
  a.code_stride = c->code_stride;
  a.norm = c->norm;
  a.lr_us = L.lr_us;
  a.lr_vt = L.lr_vt;
  a.lr_u = L.lr_u;
  return a;
}

}  // namespace

SAI_API void sai_tqcache_destroy(sai_tqcache* c) {
  if (!c) return;
  for (auto& L : c->layers) {
    for (void* p : {(void*)L.codes_k, (void*)L.codes_v, (void*)L.par_k, (void*)L.par_v,
                    (void*)L.sg_k, (void*)L.sg_v, (void*)L.rot, (void*)L.lr_us, (void*)L.lr_vt,
                    (void*)L.lr_u})
      if (p) (void)hipFree(p);
  }
  if (c->d_lens) (void)hipFree(c->d_lens);
  if (c->partials) (void)hipFree(c->partials);
  if (c->counters) (void)hipFree(c->counters);
  delete c;
}

SAI_API sai_status sai_tqcache_create(sai_ctx* ctx, const sai_tqcache_desc* desc,
                                      sai_tqcache** out) {
  if (!ctx || !desc || !out) return SAI_ERR_NULL;
  *out = nullptr;
  const sai_tqcache_desc& d = *desc;
  if (d.num_layers <= 0 || d.num_kv_heads <= 0 || d.max_batch <= 0 || d.max_rows <= 0)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "tq_cache: zero dimension");
  if (d.head_dim != 64 && d.head_dim != 128 && d.head_dim != 256)
    return fail(ctx, SAI_ERR_UNSUPPORTED, "tq_cache: head_dim %d (64, 128 or 256)", d.head_dim);
  if (d.bits != 3 && d.bits != 4 && d.bits != 8)
    return fail(ctx, SAI_ERR_INVALID_ATTRIBUTE, "bits must be 3, 4, or 8");
  // the write grid's y is 2 x heads (K and V), its z the sequences
  if (d.num_kv_heads > 32767 || d.max_batch > 65535)
    return fail(ctx, SAI_ERR_UNSUPPORTED, "tq_cache: more than 32767 heads or 65535 sequences");
  if (d.lowrank_k < 0)
    return fail(ctx, SAI_ERR_INVALID_ATTRIBUTE, "tq_cache: lowrank_k %d", d.lowrank_k);
  DeviceGuard dg(ctx->device);
  sai_tqcache* c = new (std::nothrow) sai_tqcache();
  if (!c) return fail(ctx, SAI_ERR_ALLOC, "tq_cache: host");
  c->desc = d;
  c->desc.qjl = d.qjl ? 1 : 0;
  c->code_stride = (((size_t)d.head_dim * d.bits / 8) + 15) / 16 * 16;
  c->rows_total = (size_t)d.num_kv_heads * d.max_batch * d.max_rows;
  c->tiles_cap = (d.max_rows + 63) / 64;
  const size_t v_bytes =
      (size_t)d.num_kv_heads * d.max_batch * c->tiles_cap * sai::tq_vtile_bytes(d.head_dim, d.bits);
  c->norm = 1.0f / sqrt_approx_newton((float)d.head_dim);
  c->layers.resize(d.num_layers);
  hipError_t e = hipSuccess;
  std::vector<int8_t> rot((size_t)d.num_kv_heads * d.head_dim);
  for (int l = 0; l < d.num_layers && e == hipSuccess; ++l) {
    sai_tqcache::Layer& L = c->layers[l];
    e = hipMalloc(&L.codes_k, c->rows_total * c->code_stride);
    if (e == hipSuccess) e = hipMalloc(&L.codes_v, v_bytes);
    if (e == hipSuccess) e = hipMalloc(&L.par_k, c->rows_total * sizeof(float4));
    if (e == hipSuccess) e = hipMalloc(&L.par_v, c->rows_total * sizeof(float4));
    if (e == hipSuccess && c->desc.qjl) e = hipMalloc(&L.sg_k, c->rows_total * d.head_dim / 8);
    if (e == hipSuccess && c->desc.qjl) e = hipMalloc(&L.sg_v, c->rows_total * d.head_dim / 8);
    if (e == hipSuccess) e = hipMalloc(&L.rot, rot.size());
    if (e == hipSuccess && d.lowrank_k > 0) e = hipMalloc(&L.lr_us, c->rows_total * sizeof(float));
    if (e == hipSuccess && d.lowrank_k > 0) e = hipMalloc(&L.lr_u, c->rows_total * sizeof(float));
    if (e == hipSuccess && d.lowrank_k > 0)
      e = hipMalloc(&L.lr_vt, (size_t)d.num_kv_heads * d.max_batch * d.head_dim * sizeof(float));
    if (e == hipSuccess) {
      for (int h = 0; h < d.num_kv_heads; ++h)
        tq_rotation_signs(d.seed, l, d.num_kv_heads, h, d.head_dim, rot.data() + (size_t)h * d.head_dim);
      e = hipMemcpy(L.rot, rot.data(), rot.size(), hipMemcpyHostToDevice);
    }
  }
  if (e == hipSuccess) e = hipMalloc(&c->d_lens, (size_t)d.max_batch * sizeof(int32_t));
  if (e == hipSuccess) e = hipMemset(c->d_lens, 0, (size_t)d.max_batch * sizeof(int32_t));
  if (e != hipSuccess) {
    sai_tqcache_destroy(c);
    return fail(ctx, SAI_ERR_ALLOC, "tq_cache: %s", hipGetErrorString(e));
  }
  c->h_lens.assign(d.max_batch, 0);
  // attention partials at the automatic split: about 768 workgroups plus one
  // rounding split per (sequence, kv head), groups up to 8 (4 at head_dim 256)
  {
    const size_t units = (size_t)d.max_batch * d.num_kv_heads;
    const size_t n = (768 + 2 * units) * (d.head_dim > 128 ? 4 : 8) * (d.head_dim + 2);
    const size_t nc = units * sizeof(int32_t);
    if (hipMalloc(&c->partials, n * sizeof(float)) != hipSuccess ||
        hipMalloc(&c->counters, nc) != hipSuccess || hipMemset(c->counters, 0, nc) != hipSuccess) {
      sai_tqcache_destroy(c);
      return fail(ctx, SAI_ERR_ALLOC, "tq_cache: workspace");
    }
    c->partial_floats = n;
  }
  *out = c;
  return SAI_OK;
}

SAI_API sai_status sai_tqcache_write(sai_ctx* ctx, sai_tqcache* c, int32_t layer, const void* k,
                                     const void* v, int32_t dtype, int32_t batch, int32_t s_new,
                                     void* stream) {
  if (!ctx || !c) return SAI_ERR_NULL;
  const char* op = "tq_cache_write";
  if (layer < 0 || layer >= c->desc.num_layers)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "%s: layer_idx %d", op, layer);
  if (dtype != SAI_DTYPE_F32 && dtype != SAI_DTYPE_BF16)
    return fail(ctx, SAI_ERR_UNSUPPORTED, "%s: dtype %d (want f32 or bf16)", op, dtype);
  if (batch <= 0 || batch > c->desc.max_batch || s_new <= 0 ||
      (int64_t)batch * s_new * c->desc.num_kv_heads * 2 > INT32_MAX)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "%s: batch %d / rows %d", op, batch, s_new);
  if (!k || !v) return fail(ctx, SAI_ERR_NULL, "%s: missing key/value", op);
  const bool fresh = c->pending == 0;
  if (!fresh && (s_new != c->pending || batch != c->batch))
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH,
                "%s: %d rows x %d sequences, but this pass appends %d x %d", op, s_new, batch,
                c->pending, c->batch);
  for (int b = 0; b < batch; ++b)
    if ((int64_t)c->h_lens[b] + s_new > c->desc.max_rows)
      return fail(ctx, SAI_ERR_OVERFLOW, "%s: position_overflow (sequence %d: %d + %d > %d)", op,
                  b, c->h_lens[b], s_new, c->desc.max_rows);
  if (c->layers[layer].lr_written)
    return fail(ctx, SAI_ERR_UNSUPPORTED,
                "%s: layer %d's low-rank K already took this pass's rows", op, layer);
  DeviceGuard dg(ctx->device);
  sai::TqArgs a = tq_args(c, layer);
  const int bf = dtype == SAI_DTYPE_BF16 ? 1 : 0;
  hipError_t e = sai::launch_tq_write(a, k, v, bf, batch, s_new, (hipStream_t)stream);
  if (e == hipSuccess && a.lr_us)
    e = sai::launch_tq_lowrank(a, k, bf, batch, s_new, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "tq_cache_write launch");
  if (a.lr_us) c->layers[layer].lr_written = true;
  c->pending = s_new;
  c->batch = batch;
  return SAI_OK;
}

SAI_API sai_status sai_tqcache_advance(sai_ctx* ctx, sai_tqcache* c, void* stream) {
  if (!ctx || !c) return SAI_ERR_NULL;
  if (c->pending == 0) return SAI_OK;
  DeviceGuard dg(ctx->device);
  const hipError_t e = sai::launch_seq_advance(c->d_lens, c->batch, c->pending, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "tq_cache_advance");
  for (int b = 0; b < c->batch; ++b) c->h_lens[b] += c->pending;
  c->pending = 0;
  for (auto& L : c->layers) L.lr_written = false;
  return SAI_OK;
}

SAI_API sai_status sai_tqcache_reset(sai_ctx* ctx, sai_tqcache* c) {
  if (!ctx || !c) return SAI_ERR_NULL;
  DeviceGuard dg(ctx->device);
  // synchronous: after every launch already enqueued on any stream
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemset(c->d_lens, 0, (size_t)c->desc.max_batch * sizeof(int32_t));
  if (e != hipSuccess) return hip_fail(ctx, e, "tq_cache_reset");
  std::fill(c->h_lens.begin(), c->h_lens.end(), 0);
  c->pending = 0;
  c->batch = 0;
  for (auto& L : c->layers) L.lr_written = false;
  return SAI_OK;
}

SAI_API sai_status sai_tqcache_set_lengths(sai_ctx* ctx, sai_tqcache* c, const int32_t* lens,
                                           int32_t batch) {
  if (!ctx || !c || !lens) return SAI_ERR_NULL;
  if (batch <= 0 || batch > c->desc.max_batch)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "tq_cache_set_lengths: batch %d", batch);
  if (c->desc.lowrank_k > 0)
    return fail(ctx, SAI_ERR_UNSUPPORTED,
                "tq_cache_set_lengths: the low-rank K state follows the rows written; reset instead");
  for (int b = 0; b < batch; ++b)
    if (lens[b] < 0 || lens[b] > c->desc.max_rows)
      return fail(ctx, SAI_ERR_OVERFLOW, "tq_cache_set_lengths: length %d of sequence %d exceeds %d",
                  lens[b], b, c->desc.max_rows);
  DeviceGuard dg(ctx->device);
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess)
    e = hipMemcpy(c->d_lens, lens, (size_t)batch * sizeof(int32_t), hipMemcpyHostToDevice);
  if (e != hipSuccess) return hip_fail(ctx, e, "tq_cache_set_lengths");
  std::copy(lens, lens + batch, c->h_lens.begin());
  c->pending = 0;
  c->batch = batch;
  return SAI_OK;
}

SAI_API sai_status sai_tqcache_lengths(const sai_tqcache* c, int32_t* lens_out,
                                       int32_t* pending_out, int32_t* batch_out) {
  if (!c) return SAI_ERR_NULL;
  if (lens_out)
    for (int b = 0; b < c->desc.max_batch; ++b) lens_out[b] = c->h_lens[b];
  if (pending_out) *pending_out = c->pending;
  if (batch_out) *batch_out = c->batch;
  return SAI_OK;
}

SAI_API sai_status sai_tqcache_memory_bytes(const sai_tqcache* c, uint64_t* reference_bytes,
                                            uint64_t* device_bytes) {
  if (!c) return SAI_ERR_NULL;
  const sai_tqcache_desc& d = c->desc;
  if (reference_bytes) {
    // QuantizedBlock: packed data + 4 floats + dim + bits; QJLResidual: sign
    // words + c + dim (kv_compression.rs:166-168, :352-354), K and V
    const uint64_t block = ((uint64_t)d.head_dim * d.bits + 7) / 8 + 4 * 4 + 8 + 1;
    const uint64_t resid = ((uint64_t)d.head_dim + 63) / 64 * 8 + 4 + 8;
    const uint64_t per_row = 2 * block + (d.qjl ? 2 * resid : 0);
    uint64_t rows = 0, started = 0;
    for (int b = 0; b < d.max_batch; ++b) {
      rows += (uint64_t)c->h_lens[b];
      started += c->h_lens[b] > 0 ? 1 : 0;
    }
    *reference_bytes = rows * (uint64_t)d.num_layers * d.num_kv_heads * per_row;
    // LowRankK::memory_bytes (:441-444): (rows * 1 + 1 * D) floats + 32 per
    // (layer, head) holding rows
    if (d.lowrank_k > 0)
      *reference_bytes += (uint64_t)d.num_layers * d.num_kv_heads *
                          (rows * 4 + started * ((uint64_t)d.head_dim * 4 + 32));
  }
  if (device_bytes) {
    const uint64_t per_layer =
        (uint64_t)c->rows_total * (c->code_stride + 2 * sizeof(float4) +
                                   (d.qjl ? 2 * (uint64_t)d.head_dim / 8 : 0)) +
        (uint64_t)d.num_kv_heads * d.max_batch * c->tiles_cap *
            sai::tq_vtile_bytes(d.head_dim, d.bits) +
        (uint64_t)d.num_kv_heads * d.head_dim +
        (d.lowrank_k > 0 ? (uint64_t)c->rows_total * 8 +
                               (uint64_t)d.num_kv_heads * d.max_batch * d.head_dim * 4
                         : 0);
    *device_bytes = per_layer * d.num_layers + (uint64_t)d.max_batch * sizeof(int32_t);
  }
  return SAI_OK;
}

SAI_API sai_status sai_tqcache_read(sai_ctx* ctx, sai_tqcache* c, int32_t layer, int32_t b,
                                    int32_t head, int32_t start, int32_t len, float* k_out,
                                    float* v_out) {
  if (!ctx || !c) return SAI_ERR_NULL;
  const char* op = "tq_cache_read";
  if (layer < 0 || layer >= c->desc.num_layers || b < 0 || b >= c->desc.max_batch || head < 0 ||
      head >= c->desc.num_kv_heads || start < 0 || len < 0 ||
      (int64_t)start + len > (int64_t)c->h_lens[b] + (b < c->batch ? c->pending : 0))
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "%s: range out of the written rows", op);
  if (len == 0) return SAI_OK;
  if (!k_out || !v_out) return fail(ctx, SAI_ERR_NULL, "%s: NULL output", op);
  DeviceGuard dg(ctx->device);
  const size_t n = (size_t)len * c->desc.head_dim;
  float* dk = nullptr;
  // synchronous: the rows of every write already enqueued on any stream
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(ctx, e, op);
  e = hipMalloc(&dk, 2 * n * sizeof(float));
  if (e != hipSuccess) return fail(ctx, SAI_ERR_ALLOC, "%s: %s", op, hipGetErrorString(e));
  sai::TqArgs a = tq_args(c, layer);
  e = sai::launch_tq_read(a, b, head, start, len, dk, dk + n, nullptr);
  if (e == hipSuccess) e = hipMemcpy(k_out, dk, n * sizeof(float), hipMemcpyDeviceToHost);
  if (e == hipSuccess) e = hipMemcpy(v_out, dk + n, n * sizeof(float), hipMemcpyDeviceToHost);
  (void)hipFree(dk);
  if (e != hipSuccess) return hip_fail(ctx, e, op);
  return SAI_OK;
}

SAI_API sai_status sai_tqcache_read_lowrank(sai_ctx* ctx, sai_tqcache* c, int32_t layer,
                                            int32_t b, int32_t head, int32_t start, int32_t len,
                                            float* u_s, float* vt) {
  if (!ctx || !c) return SAI_ERR_NULL;
  const char* op = "tq_cache_read_lowrank";
  if (c->desc.lowrank_k <= 0) return fail(ctx, SAI_ERR_UNSUPPORTED, "%s: no low-rank K", op);
  if (layer < 0 || layer >= c->desc.num_layers || b < 0 || b >= c->desc.max_batch || head < 0 ||
      head >= c->desc.num_kv_heads || start < 0 || len < 0 ||
      (int64_t)start + len > (int64_t)c->h_lens[b] + (b < c->batch ? c->pending : 0))
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "%s: range out of the written rows", op);
  DeviceGuard dg(ctx->device);
  const sai_tqcache::Layer& L = c->layers[layer];
  const size_t hb = (size_t)head * c->desc.max_batch + b;
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess && u_s && len > 0)
    e = hipMemcpy(u_s, L.lr_us + hb * c->desc.max_rows + start, (size_t)len * sizeof(float),
                  hipMemcpyDeviceToHost);
  if (e == hipSuccess && vt)
    e = hipMemcpy(vt, L.lr_vt + hb * c->desc.head_dim, (size_t)c->desc.head_dim * sizeof(float),
                  hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(ctx, e, op);
  return SAI_OK;
}

SAI_API sai_status sai_tqcache_read_raw(sai_ctx* ctx, sai_tqcache* c, int32_t layer, int32_t b,
                                        int32_t head, int32_t start, int32_t len, void* k_codes,
                                        void* v_codes, float* k_params, float* v_params,
                                        void* k_signs, void* v_signs) {
  if (!ctx || !c) return SAI_ERR_NULL;
  const char* op = "tq_cache_read_raw";
  if (layer < 0 || layer >= c->desc.num_layers || b < 0 || b >= c->desc.max_batch || head < 0 ||
      head >= c->desc.num_kv_heads || start < 0 || len < 0 ||
      (int64_t)start + len > (int64_t)c->h_lens[b] + (b < c->batch ? c->pending : 0))
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "%s: range out of the written rows", op);
  if (len == 0) return SAI_OK;
  DeviceGuard dg(ctx->device);
  {
    // synchronous: the rows of every write already enqueued on any stream
    const hipError_t es = hipDeviceSynchronize();
    if (es != hipSuccess) return hip_fail(ctx, es, op);
  }
  const sai_tqcache::Layer& L = c->layers[layer];
  const size_t row0 = ((size_t)head * c->desc.max_batch + b) * c->desc.max_rows + start;
  const size_t cb = (size_t)c->desc.head_dim * c->desc.bits / 8;
  hipError_t e = hipSuccess;
  auto codes = [&](const uint8_t* src, void* dst) {
    if (!dst || e != hipSuccess) return;
    e = hipMemcpy2D(dst, cb, src + row0 * c->code_stride, c->code_stride, cb, len,
                    hipMemcpyDeviceToHost);
  };
  // V: the tiles covering the rows, repacked row-major (LSB first)
  auto vcodes = [&](const uint8_t* src, void* dst) {
    if (!dst || e != hipSuccess) return;
    const int D = c->desc.head_dim, B = c->desc.bits;
    const size_t tb = sai::tq_vtile_bytes(D, B);
    const int t0 = start / 64, t1 = (start + len - 1) / 64;
    std::vector<uint32_t> tiles((size_t)(t1 - t0 + 1) * tb / 4);
    e = hipMemcpy(tiles.data(),
                  src + (((size_t)head * c->desc.max_batch + b) * c->tiles_cap + t0) * tb,
                  tiles.size() * 4, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return;
    uint8_t* out = (uint8_t*)dst;
    std::fill(out, out + (size_t)len * cb, 0);
    for (int t = 0; t < len; ++t) {
      const int r = start + t;
      const uint32_t* tw = tiles.data() + (size_t)(r / 64 - t0) * (tb / 4);
      for (int d = 0; d < D; ++d) {
        const uint32_t* ew = tw + (size_t)d * 2 * B;
        const int p = (r % 64) * B, w = p >> 5, sh = p & 31;
        uint32_t code = ew[w] >> sh;
        if (sh + B > 32) code |= ew[w + 1] << (32 - sh);
        code &= (1u << B) - 1u;
        for (int k = 0; k < B; ++k)
          if (code >> k & 1u) out[(size_t)t * cb + (d * B + k) / 8] |= (uint8_t)(1u << ((d * B + k) % 8));
      }
    }
  };
  auto params = [&](const float4* src, float* dst) {
    if (!dst || e != hipSuccess) return;
    std::vector<float4> tmp(len);
    e = hipMemcpy(tmp.data(), src + row0, len * sizeof(float4), hipMemcpyDeviceToHost);
    for (int t = 0; t < len && e == hipSuccess; ++t) {
      dst[3 * t] = tmp[t].x;
      dst[3 * t + 1] = tmp[t].y;
      dst[3 * t + 2] = tmp[t].z;
    }
  };
  auto signs = [&](const uint32_t* src, void* dst) {
    if (!dst || !src || e != hipSuccess) return;
    e = hipMemcpy(dst, src + row0 * (c->desc.head_dim / 32), (size_t)len * c->desc.head_dim / 8,
                  hipMemcpyDeviceToHost);
  };
  codes(L.codes_k, k_codes);
  vcodes(L.codes_v, v_codes);
  params(L.par_k, k_params);
  params(L.par_v, v_params);
  signs(L.sg_k, k_signs);
  signs(L.sg_v, v_signs);
  if (e != hipSuccess) return hip_fail(ctx, e, op);
  return SAI_OK;
}

namespace {

// The three read paths over a TurboQuant layer: mode 0 attention, 1 logits,
// 2 weighted value sum. q / weights / out as the entry points document.
sai_status tq_read_path(sai_ctx* ctx, sai_tqcache* c, int32_t layer, int mode, const void* q,
                        int32_t dtype, const float* weights, int32_t ld, int32_t batch,
                        int32_t num_heads, float scale_log2, float* out, void* stream,
                        const char* op, const void* k_new = nullptr, const void* v_new = nullptr,
                        int32_t kv_dtype = SAI_DTYPE_F32) {
  if (mode != 2 && !q) return fail(ctx, SAI_ERR_NULL, "%s: missing query", op);
  if (mode == 2 && !weights) return fail(ctx, SAI_ERR_NULL, "%s: missing weights", op);
  if (!out) return fail(ctx, SAI_ERR_NULL, "%s: missing output", op);
  if (layer < 0 || layer >= c->desc.num_layers)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "%s: layer_idx %d", op, layer);
  if (mode != 2 && dtype != SAI_DTYPE_F32 && dtype != SAI_DTYPE_BF16)
    return fail(ctx, SAI_ERR_UNSUPPORTED, "%s: dtype %d (want f32 or bf16)", op, dtype);
  const int H = c->desc.num_kv_heads, D = c->desc.head_dim;
  if (num_heads <= 0 || num_heads % H != 0)
    return fail(ctx, SAI_ERR_INVALID_ATTRIBUTE,
                "GroupQueryAttention: num_heads must be a multiple of kv_num_heads");
  const int G = num_heads / H;
  if (G != 1 && G != 2 && G != 4 && G != 8)
    return fail(ctx, SAI_ERR_UNSUPPORTED, "%s: group size %d (supported 1, 2, 4, 8)", op, G);
  if (D == 256 && G > 4)
    return fail(ctx, SAI_ERR_UNSUPPORTED, "%s: head_dim 256 supports groups of 1, 2 and 4", op);
  const int nb = c->pending > 0 ? c->batch : batch;
  if (batch <= 0 || batch != nb || batch > c->desc.max_batch)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "%s: batch %d does not match the cache's %d", op,
                batch, nb);
  int32_t max_len = 0;
  for (int b = 0; b < batch; ++b) max_len = std::max(max_len, c->h_lens[b] + c->pending);
  if (max_len <= 0) return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "%s: empty cache", op);
  if (mode != 0 && ld < max_len)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "%s: row stride %d below the %d positions", op, ld,
                max_len);
  // automatic split: about one workgroup per CU (256; 8 waves each up to
  // head_dim 128, 4 at 256), in multiples of one 64-position tile per wave.
  // A second workgroup on a CU starts its stream late: its loads queue behind
  // the first one's. At 16 x 8192 x 8 kv heads, streamed from HBM, 2 splits of
  // 8 waves measured 40.1 us per step against 44.3 for 4 splits of 4 waves.
  int32_t split_rows = ctx->tq_split;
  if (split_rows <= 0) {
    const int64_t units = (int64_t)batch * H;
    const int64_t quantum = D <= 128 ? 512 : 256;
    const int64_t want = std::max<int64_t>(
        1, std::min<int64_t>((256 + units - 1) / units, (max_len + quantum - 1) / quantum));
    split_rows = (int32_t)(((max_len + want - 1) / want + quantum - 1) / quantum * quantum);
    // up to head_dim 128, more than 8 splits per sequence: two tiles per wave
    // at least (1 x 8192 positions, 8 kv heads: 14.08 -> 13.72 us per step;
    // 1 x 16384, 1 kv head: 21.76 -> 20.12 us; 2 x 3000 keeps 512: 13.2
    // against 13.6 at 1024)
    if (D <= 128 && want > 8) split_rows = std::max<int32_t>(split_rows, 1024);
  }
  const int32_t max_splits = (max_len + split_rows - 1) / split_rows;
  const size_t part_floats = (size_t)batch * H * max_splits * G * (D + 2);
  DeviceGuard dg(ctx->device);
  // the cache's partials are sized at creation for the automatic split; a
  // smaller split set for tuning may grow them once, after the device is idle
  if (mode != 1 && part_floats > c->partial_floats) {
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return hip_fail(ctx, e, op);
    if (c->partials) (void)hipFree(c->partials);
    c->partials = nullptr;
    c->partial_floats = 0;
    if (hipMalloc(&c->partials, part_floats * sizeof(float)) != hipSuccess)
      return fail(ctx, SAI_ERR_ALLOC, "%s: workspace", op);
    c->partial_floats = part_floats;
  }
  sai::TqArgs a = tq_args(c, layer);
  sai::TqAttendArgs t{};
  t.q = q;
  t.q_bf16 = dtype == SAI_DTYPE_BF16 ? 1 : 0;
  t.num_heads = num_heads;
  t.out = out;
  t.partials = c->partials;
  t.counters = c->counters;
  t.weights = weights;
  t.ld = ld;
  t.normalize = mode == 0 ? 1 : 0;
  t.k_new = k_new;
  t.v_new = v_new;
  t.kv_bf16 = kv_dtype == SAI_DTYPE_BF16 ? 1 : 0;
  t.split_rows = split_rows;
  t.max_splits = max_splits;
  t.scale_log2 = scale_log2;
  t.static_tiles = ctx->reproducible == 1;
  const hipError_t e =
      sai::launch_tq_attend(a, t, mode, G, max_splits, batch, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(ctx, e, op);
  return SAI_OK;
}

}  // namespace

SAI_API sai_status sai_tqcache_attend(sai_ctx* ctx, sai_tqcache* c, int32_t layer, const void* q,
                                      int32_t dtype, int32_t batch, int32_t num_heads,
                                      int32_t has_scale, float scale, float* out, void* stream) {
  if (!ctx || !c) return SAI_ERR_NULL;
  const float sc = has_scale ? scale : sai_default_scale(c->desc.head_dim);
  return tq_read_path(ctx, c, layer, 0, q, dtype, nullptr, 0, batch, num_heads,
                      sc * 1.4426950408889634f, out, stream, "tq_cache_attend");
}

SAI_API sai_status sai_tqcache_write_attend(sai_ctx* ctx, sai_tqcache* c, int32_t layer,
                                            const void* q, int32_t q_dtype, const void* k_new,
                                            const void* v_new, int32_t kv_dtype, int32_t batch,
                                            int32_t num_heads, int32_t has_scale, float scale,
                                            float* out, void* stream) {
  if (!ctx || !c) return SAI_ERR_NULL;
  const char* op = "tq_cache_write_attend";
  if (!k_new || !v_new) return fail(ctx, SAI_ERR_NULL, "%s: missing key/value", op);
  if (layer < 0 || layer >= c->desc.num_layers)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "%s: layer_idx %d", op, layer);
  if (kv_dtype != SAI_DTYPE_F32 && kv_dtype != SAI_DTYPE_BF16)
    return fail(ctx, SAI_ERR_UNSUPPORTED, "%s: dtype %d (want f32 or bf16)", op, kv_dtype);
  if (batch <= 0 || batch > c->desc.max_batch)
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH, "%s: batch %d", op, batch);
  if (c->pending != 0 && (c->pending != 1 || batch != c->batch))
    return fail(ctx, SAI_ERR_SHAPE_MISMATCH,
                "%s: 1 row x %d sequences, but this pass appends %d x %d", op, batch, c->pending,
                c->batch);
  for (int b = 0; b < batch; ++b)
    if ((int64_t)c->h_lens[b] + 1 > c->desc.max_rows)
      return fail(ctx, SAI_ERR_OVERFLOW, "%s: position_overflow (sequence %d: %d + 1 > %d)", op,
                  b, c->h_lens[b], c->desc.max_rows);
  if (c->layers[layer].lr_written)
    return fail(ctx, SAI_ERR_UNSUPPORTED,
                "%s: layer %d's low-rank K already took this pass's rows", op, layer);
  const int32_t pending = c->pending, pbatch = c->batch;
  c->pending = 1;
  c->batch = batch;
  const float sc = has_scale ? scale : sai_default_scale(c->desc.head_dim);
  sai_status st = tq_read_path(ctx, c, layer, 0, q, q_dtype, nullptr, 0, batch, num_heads,
                               sc * 1.4426950408889634f, out, stream, op, k_new, v_new, kv_dtype);
  if (st == SAI_OK && c->layers[layer].lr_us) {
    const hipError_t e = sai::launch_tq_lowrank(tq_args(c, layer), k_new,
                                                kv_dtype == SAI_DTYPE_BF16 ? 1 : 0, batch, 1,
                                                (hipStream_t)stream);
    if (e != hipSuccess) st = hip_fail(ctx, e, op);
    else c->layers[layer].lr_written = true;
  }
  if (st != SAI_OK) {
    c->pending = pending;
    c->batch = pbatch;
  }
  return st;
}

SAI_API sai_status sai_tqcache_attention_logits(sai_ctx* ctx, sai_tqcache* c, int32_t layer,
                                                const void* q, int32_t dtype, int32_t batch,
                                                int32_t num_heads, float* logits, int32_t ld,
                                                void* stream) {
  if (!ctx || !c) return SAI_ERR_NULL;
  return tq_read_path(ctx, c, layer, 1, q, dtype, nullptr, ld, batch, num_heads, 1.0f, logits,
                      stream, "tq_cache_attention_logits");
}

SAI_API sai_status sai_tqcache_weighted_value_sum(sai_ctx* ctx, sai_tqcache* c, int32_t layer,
                                                  const float* weights, int32_t ld,
                                                  int32_t batch, int32_t num_heads, float* out,
                                                  void* stream) {
  if (!ctx || !c) return SAI_ERR_NULL;
  return tq_read_path(ctx, c, layer, 2, nullptr, SAI_DTYPE_F32, weights, ld, batch, num_heads,
                      1.0f, out, stream, "tq_cache_weighted_value_sum");
}
