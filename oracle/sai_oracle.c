/*
 * CPU oracle for the compressed-KV GroupQueryAttention path.
 *
 * TEST INFRASTRUCTURE ONLY -- the checker, never the product. Only tests/,
 * the smoke entry and bench.py's CPU-baseline leg load it.
 *
 * A C restatement of the reference's Rust CPU semantics, op for op. Each
 * function names the reference file:line it follows (paths relative to the
 * reference workspace root). Build flags: -O2 -ffp-contract=off
 * -fno-fast-math, so that every f32 multiply and add rounds on its own, as
 * in Rust.
 *
 * Parity status of each function (how it is pinned) is recorded in the
 * header comment of tests/test_oracle.py next to the tests that pin it.
 */
#include "sai_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define OK 0
#define ERR_INVALID_ATTRIBUTE (-1)
#define ERR_SHAPE_MISMATCH (-2)

static inline uint32_t f2u(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}
static inline float u2f(uint32_t u) {
  float x;
  memcpy(&x, &u, 4);
  return x;
}

/* ------------------------------------------------------------------------
 * Rust `as` casts from f32 (saturating, NaN -> 0).
 * ---------------------------------------------------------------------- */
int32_t sai_or_sat_i32(float x) {
  if (x != x) return 0;
  if (x >= 2147483648.0f) return INT32_MAX;
  if (x <= -2147483648.0f) return INT32_MIN;
  return (int32_t)x;
}

uint32_t sai_or_sat_u32(float x) {
  if (x != x) return 0;
  if (x <= 0.0f) return 0;
  if (x >= 4294967296.0f) return UINT32_MAX;
  return (uint32_t)x;
}

int64_t sai_or_sat_i64(float x) {
  if (x != x) return 0;
  if (x >= 9223372036854775808.0f) return INT64_MAX;
  if (x <= -9223372036854775808.0f) return INT64_MIN;
  return (int64_t)x;
}

/* ------------------------------------------------------------------------
 * expf_approx -- onnx-rt/src/operators.rs:1311-1357.
 * Clamp to +-88.7, k = nearest integer of x*log2(e) (half away from zero via
 * `(t +- 0.5) as i32`), f = x - k*ln2, degree-4 Taylor polynomial evaluated
 * left to right, times 2^k built from exponent bits; k+127 < 0 -> 0.
 * ---------------------------------------------------------------------- */
float sai_or_expf_approx(float x) {
  const float clamp_max = 88.7f;
  const float clamp_min = -88.7f;
  const float c2 = 0.5f;
  const float c3 = 1.0f / 6.0f;
  const float c4 = 1.0f / 24.0f;
  const float log2_e = 1.44269504088896340736f; /* core::f32::consts::LOG2_E */
  const float ln_2 = 0.693147180559945309417f;  /* core::f32::consts::LN_2 */
  /* f32::clamp: NaN passes through. */
  if (x < clamp_min) x = clamp_min;
  if (x > clamp_max) x = clamp_max;
  float t = x * log2_e;
  int32_t k = (t >= 0.0f) ? sai_or_sat_i32(t + 0.5f) : sai_or_sat_i32(t - 0.5f);
  if ((int64_t)k + 127 < 0) return 0.0f;
  float f = x - ((float)k) * ln_2;
  float f2 = f * f;
  float p = 1.0f + f + f2 * c2 + f2 * f * c3 + f2 * f2 * c4;
  uint32_t bits = ((uint32_t)(k + 127)) << 23;
  return p * u2f(bits);
}

void sai_or_expf_approx_array(const float* x, size_t n, float* out) {
  for (size_t i = 0; i < n; ++i) out[i] = sai_or_expf_approx(x[i]);
}

/* sqrt_f32 -- onnx-rt/src/ops/microsoft.rs:54-63 (16 Newton steps). */
float sai_or_sqrt_f32(float x) {
  if (x <= 0.0f) return 0.0f;
  float guess = x;
  for (int i = 0; i < 16; ++i) guess = 0.5f * (guess + x / guess);
  return guess;
}

/* sqrt_approx -- onnx-rt/src/operators.rs:3311-3320 (10 Newton steps). */
float sai_or_sqrt_approx(float x) {
  if (x <= 0.0f) return 0.0f;
  float s = x;
  for (int i = 0; i < 10; ++i) s = 0.5f * (s + x / s);
  return s;
}

/* Default attention scale of GQA: 1 / sqrt_f32(head_dim)
 * (onnx-rt/src/ops/microsoft.rs:1153). */
float sai_or_default_scale(int head_dim) {
  return 1.0f / sai_or_sqrt_f32((float)head_dim);
}

/* round_half_even -- onnx-rt/src/ops/quantized.rs:33-50. */
float sai_or_round_half_even(float x) {
  float i = (float)sai_or_sat_i64(x);
  float f = (x < 0.0f && i != x) ? i - 1.0f : i;
  float frac = x - f;
  if (frac < 0.5f) return f;
  if (frac > 0.5f) return f + 1.0f;
  int64_t fi = sai_or_sat_i64(f);
  return ((fi & 1) == 0) ? f : f + 1.0f;
}

void sai_or_round_half_even_array(const float* x, size_t n, float* out) {
  for (size_t i = 0; i < n; ++i) out[i] = sai_or_round_half_even(x[i]);
}

/* round_f32 (half away from zero) -- onnx-rt/src/kv_compression.rs:27-37. */
float sai_or_round_f32_kv(float x) {
  float trunc = (float)sai_or_sat_i32(x);
  float frac = x - trunc;
  if (frac >= 0.5f) return trunc + 1.0f;
  if (frac <= -0.5f) return trunc - 1.0f;
  return trunc;
}

/* f32_to_bf16 / bf16_to_f32 -- onnx-rt/src/tensor.rs:312-329, 293-305. */
uint16_t sai_or_f32_to_bf16(float x) {
  uint32_t bits = f2u(x);
  if (x != x) return (uint16_t)((bits >> 16) | 0x0040u);
  uint32_t bias = 0x00007FFFu + ((bits >> 16) & 1u);
  return (uint16_t)((bits + bias) >> 16);
}

float sai_or_bf16_to_f32(uint16_t b) { return u2f(((uint32_t)b) << 16); }

/* IEEE 754 binary32 -> binary16, round to nearest even, overflow to inf,
 * gradual underflow. The reference has no f16 type; the int4 KV spec stores
 * its scale and zero point as binary16, so this follows IEEE 754-2008 5.4.2. */
uint16_t sai_or_f32_to_f16(float x) {
  uint32_t b = f2u(x);
  uint32_t sign = (b >> 16) & 0x8000u;
  uint32_t e = (b >> 23) & 0xFFu;
  uint32_t m = b & 0x7FFFFFu;
  if (e == 0xFFu) {
    if (m == 0) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | 0x7E00u | (m >> 13));
  }
  if (e == 0) return (uint16_t)sign; /* f32 zero/subnormal: far below 2^-25 */
  int32_t E = (int32_t)e - 127;
  if (E > 15) return (uint16_t)(sign | 0x7C00u);
  uint32_t mant = m | 0x800000u; /* 24 significant bits */
  if (E >= -14) {
    uint32_t h = ((uint32_t)(E + 15) << 10) | (m >> 13);
    uint32_t r = m & 0x1FFFu;
    if (r > 0x1000u || (r == 0x1000u && (h & 1u))) h += 1u; /* carry may reach inf */
    return (uint16_t)(sign | h);
  }
  /* subnormal binary16: value = mant * 2^(E-23), unit 2^-24 */
  int32_t shift = -E - 1; /* >= 14 */
  if (shift >= 26) return (uint16_t)sign; /* < 2^-26 rounds to zero */
  uint32_t q = mant >> shift;
  uint32_t r = mant & ((1u << shift) - 1u);
  uint32_t half = 1u << (shift - 1);
  if (r > half || (r == half && (q & 1u))) q += 1u;
  return (uint16_t)(sign | q);
}

float sai_or_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = ((uint32_t)h >> 10) & 0x1Fu;
  uint32_t m = (uint32_t)h & 0x3FFu;
  if (e == 0x1Fu) return u2f(sign | 0x7F800000u | (m << 13));
  if (e == 0) {
    /* zero or subnormal: m * 2^-24, exact in f32 */
    float v = (float)m * (1.0f / 16777216.0f);
    return (sign ? -v : v);
  }
  return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

void sai_or_f32_to_f16_array(const float* x, size_t n, uint16_t* out) {
  for (size_t i = 0; i < n; ++i) out[i] = sai_or_f32_to_f16(x[i]);
}

/* pack_bits / unpack_bits -- onnx-rt/src/kv_compression.rs:294-333
 * (LSB-first: bit b of value i lands at stream bit i*bits+b). */
void sai_or_pack_bits(const uint32_t* values, size_t n, int bits, uint8_t* out) {
  size_t nbytes = (n * (size_t)bits + 7) / 8;
  memset(out, 0, nbytes);
  size_t pos = 0;
  for (size_t i = 0; i < n; ++i) {
    for (int b = 0; b < bits; ++b) {
      if ((values[i] >> b) & 1u) out[pos / 8] |= (uint8_t)(1u << (pos % 8));
      ++pos;
    }
  }
}

void sai_or_unpack_bits(const uint8_t* data, size_t nbytes, size_t count, int bits,
                        uint32_t* out) {
  size_t pos = 0;
  for (size_t i = 0; i < count; ++i) {
    uint32_t v = 0;
    for (int b = 0; b < bits; ++b) {
      size_t byte = pos / 8, bit = pos % 8;
      if (byte < nbytes && ((data[byte] >> bit) & 1u)) v |= 1u << b;
      ++pos;
    }
    out[i] = v;
  }
}

/* ------------------------------------------------------------------------
 * RoPE tables of the Gemma loader: precompute_rope_tables
 * (onnx-rt/src/model_loader/gemma.rs:458-472) with powf_approx (:480-483),
 * ln_approx (:485-500), exp_approx (:502-513), libm_floor_f32 (:517-524),
 * sin_approx (:526-535), cos_approx (:537-539). Every step is one f32
 * operation, rounded on its own, in the reference's order; the constants are
 * Rust's core::f32::consts, written here as decimal literals that the
 * compiler rounds to the same f32 values.
 * ---------------------------------------------------------------------- */
#define OR_LN_2 0.693147180559945309417232121458176568f
#define OR_LOG2_E 1.44269504088896340735992468100189214f
#define OR_TAU 6.28318530717958647692528676655900577f
#define OR_PI 3.14159265358979323846264338327950288f
#define OR_FRAC_PI_2 1.57079632679489661923132169163975144f

float sai_or_floor_approx(float x) {
  float xi = (float)sai_or_sat_i32(x); /* `x as i32 as f32` */
  return x < xi ? xi - 1.0f : xi;
}

float sai_or_ln_approx(float x) {
  if (x <= 0.0f) return -INFINITY;
  uint32_t bits = f2u(x);
  int32_t e = (int32_t)((bits >> 23) & 0xffu) - 127;
  float m = u2f((bits & 0x7fffffu) | (127u << 23));
  float y = (m - 1.0f) / (m + 1.0f);
  float y2 = y * y;
  float acc = y + y2 * y / 3.0f;
  acc = acc + y2 * y2 * y / 5.0f;
  acc = acc + y2 * y2 * y2 * y / 7.0f;
  float ln_m = 2.0f * acc;
  return (float)e * OR_LN_2 + ln_m;
}

float sai_or_exp_approx(float x) {
  float y = x * OR_LOG2_E;
  int32_t k = sai_or_sat_i32(sai_or_floor_approx(y));
  float r = x - (float)k * OR_LN_2;
  float p = 1.0f / 24.0f + r * (1.0f / 120.0f);
  p = 1.0f / 6.0f + r * p;
  p = 0.5f + r * p;
  p = 1.0f + r * p;
  float e_r = 1.0f + r * p;
  int32_t kc = k < -126 ? -126 : (k > 127 ? 127 : k);
  float two_k = u2f((uint32_t)(kc + 127) << 23);
  return e_r * two_k;
}

float sai_or_sin_approx(float x) {
  float y = x - sai_or_floor_approx(x / OR_TAU) * OR_TAU;
  if (y > OR_PI) y -= OR_TAU;
  float y2 = y * y;
  float p = 1.0f / 5040.0f - y2 * (1.0f / 362880.0f);
  p = 1.0f / 120.0f - y2 * p;
  p = 1.0f / 6.0f - y2 * p;
  p = 1.0f - y2 * p;
  return y * p;
}

float sai_or_cos_approx(float x) { return sai_or_sin_approx(x + OR_FRAC_PI_2); }

void sai_or_rope_tables_bf16(int max_pos, int half, float rope_theta, uint16_t* cos_out,
                             uint16_t* sin_out) {
  float head_dim = (float)(half * 2);
  for (int pos = 0; pos < max_pos; ++pos)
    for (int i = 0; i < half; ++i) {
      float ex = (2.0f * (float)i) / head_dim;
      float inv_freq = 1.0f / sai_or_exp_approx(ex * sai_or_ln_approx(rope_theta));
      float angle = (float)pos * inv_freq;
      size_t o = (size_t)pos * half + i;
      cos_out[o] = sai_or_f32_to_bf16(sai_or_cos_approx(angle));
      sin_out[o] = sai_or_f32_to_bf16(sai_or_sin_approx(angle));
    }
}

/* ------------------------------------------------------------------------
 * RoPE -- apply_rope_in_place (onnx-rt/src/ops/microsoft.rs:177-233) with
 * validate_rope_caches (:71-110), rope_position_for (:115-121),
 * check_rope_position (:125-133) and rotate_rope_block (:137-160).
 * x is [b, heads, sq, head_dim].
 * ---------------------------------------------------------------------- */
int sai_or_apply_rope(float* x, int b, int heads, int sq, int head_dim, const float* cos_cache,
                      const float* sin_cache, int cache_rows, int cache_cols,
                      const int64_t* position_ids, int n_pos, int interleaved, int rotary_dim) {
  if (n_pos != b * sq && n_pos != sq) return ERR_SHAPE_MISMATCH;
  if (rotary_dim == 0 || rotary_dim > head_dim) return ERR_INVALID_ATTRIBUTE;
  if (rotary_dim % 2 != 0) return ERR_INVALID_ATTRIBUTE;
  int half = rotary_dim / 2;
  if (cache_cols != half) return ERR_SHAPE_MISMATCH;
  size_t head_stride = (size_t)sq * head_dim;
  size_t batch_stride = (size_t)heads * head_stride;
  for (int bi = 0; bi < b; ++bi) {
    for (int hi = 0; hi < heads; ++hi) {
      for (int qi = 0; qi < sq; ++qi) {
        int64_t pos = (n_pos == sq) ? position_ids[qi] : position_ids[(size_t)bi * sq + qi];
        if (pos < 0 || pos >= cache_rows) return ERR_SHAPE_MISMATCH;
        size_t base = bi * batch_stride + hi * head_stride + (size_t)qi * head_dim;
        for (int pair = 0; pair < half; ++pair) {
          float c = cos_cache[(size_t)pos * cache_cols + pair];
          float s = sin_cache[(size_t)pos * cache_cols + pair];
          size_t i0, i1;
          if (interleaved) {
            i0 = base + 2 * (size_t)pair;
            i1 = i0 + 1;
          } else {
            i0 = base + pair;
            i1 = base + pair + half;
          }
          float x0 = x[i0];
          float x1 = x[i1];
          x[i0] = c * x0 - s * x1;
          x[i1] = s * x0 + c * x1;
        }
      }
    }
  }
  return OK;
}

/* ------------------------------------------------------------------------
 * SDPA -- scaled_dot_product_attention (onnx-rt/src/ops/microsoft.rs:380-438)
 * with sdpa_scores_row (:241-265), sdpa_softmax (:270-299),
 * sdpa_write_weighted_v (:302-319), sdpa_write_zero_row (:322-326),
 * sdpa_max_k (:331-337), sdpa_row (:341-359).
 * q [B,Hq,Sq,D], k/v [B,Hk,Sk,D], out [B,Hq,Sq,D].
 * ---------------------------------------------------------------------- */
/* Key visibility with the reference's two window rules, for the query at
 * absolute position q_pos (query qi of a chunk after past_sk cached keys):
 *  - the GPU mask (gqa_softmax_mask_f32, cuda/kernels/attention.rs:79, :111):
 *    keys k < q_pos - mask_window are hidden when mask_window > 0;
 *  - a sliding-window cache layer (GpuKvCache::view_at, cuda/kv_cache.rs:
 *    340-360): the view holds the last layer_window keys, k >= q_pos + 1 -
 *    layer_window, when layer_window > 0 (for a chunk of several queries each
 *    query's own last layer_window keys).
 * Returns the first visible key. */
static int first_visible_key(int q_pos, int layer_window, int mask_window) {
  int lo = 0;
  if (mask_window > 0 && q_pos - mask_window > lo) lo = q_pos - mask_window;
  if (layer_window > 0 && q_pos + 1 - layer_window > lo) lo = q_pos + 1 - layer_window;
  return lo;
}

static int sdpa_impl(const float* q, const float* k, const float* v, int batch, int num_q_heads,
                     int num_kv_heads, int sq, int sk, int head_dim, int past_sk, float scale,
                     int causal, int layer_window, int mask_window, float* out) {
  if (num_q_heads == 0 || num_kv_heads == 0 || head_dim == 0) return ERR_SHAPE_MISMATCH;
  if (num_q_heads % num_kv_heads != 0) return ERR_SHAPE_MISMATCH;
  int group = num_q_heads / num_kv_heads;
  size_t out_len = (size_t)batch * num_q_heads * sq * head_dim;
  memset(out, 0, out_len * sizeof(float));
  if (sk == 0) return OK;
  float* scores = (float*)malloc(sizeof(float) * (size_t)sk);
  size_t q_head_stride = (size_t)sq * head_dim;
  size_t q_batch_stride = (size_t)num_q_heads * q_head_stride;
  size_t k_head_stride = (size_t)sk * head_dim;
  size_t k_batch_stride = (size_t)num_kv_heads * k_head_stride;
  for (int bi = 0; bi < batch; ++bi) {
    for (int qh = 0; qh < num_q_heads; ++qh) {
      int kh = qh / group;
      size_t q_base = bi * q_batch_stride + qh * q_head_stride;
      size_t k_base = bi * k_batch_stride + kh * k_head_stride;
      for (int qi = 0; qi < sq; ++qi) {
        size_t q_row = q_base + (size_t)qi * head_dim;
        int max_k = causal ? ((past_sk + qi + 1) < sk ? (past_sk + qi + 1) : sk) : sk;
        int min_k = first_visible_key(past_sk + qi, layer_window, mask_window);
        /* scores */
        for (int ki = 0; ki < sk; ++ki) {
          if (ki >= max_k || ki < min_k) {
            scores[ki] = -INFINITY;
            continue;
          }
          const float* krow = k + k_base + (size_t)ki * head_dim;
          float acc = 0.0f;
          for (int d = 0; d < head_dim; ++d) acc += q[q_row + d] * krow[d];
          scores[ki] = acc * scale;
        }
        /* softmax */
        float max_val = -INFINITY;
        for (int ki = 0; ki < sk; ++ki)
          if (scores[ki] > max_val) max_val = scores[ki];
        int valid = isfinite(max_val);
        float denom = 0.0f;
        if (valid) {
          for (int ki = 0; ki < sk; ++ki) {
            float e = isfinite(scores[ki]) ? sai_or_expf_approx(scores[ki] - max_val) : 0.0f;
            denom += e;
            scores[ki] = e;
          }
          if (denom == 0.0f) valid = 0;
        }
        if (!valid) {
          for (int d = 0; d < head_dim; ++d) out[q_row + d] = 0.0f;
          continue;
        }
        float inv = 1.0f / denom;
        for (int ki = 0; ki < sk; ++ki) scores[ki] *= inv;
        /* weighted V (v_base == k_base, :421-423) */
        for (int d = 0; d < head_dim; ++d) {
          float acc = 0.0f;
          for (int ki = 0; ki < sk; ++ki) acc += scores[ki] * v[k_base + (size_t)ki * head_dim + d];
          out[q_row + d] = acc;
        }
      }
    }
  }
  free(scores);
  return OK;
}

int sai_or_sdpa(const float* q, const float* k, const float* v, int batch, int num_q_heads,
                int num_kv_heads, int sq, int sk, int head_dim, int past_sk, float scale,
                int causal, float* out) {
  return sdpa_impl(q, k, v, batch, num_q_heads, num_kv_heads, sq, sk, head_dim, past_sk, scale,
                   causal, 0, 0, out);
}

int sai_or_sdpa_window(const float* q, const float* k, const float* v, int batch,
                       int num_q_heads, int num_kv_heads, int sq, int sk, int head_dim,
                       int past_sk, float scale, int layer_window, int mask_window, float* out) {
  return sdpa_impl(q, k, v, batch, num_q_heads, num_kv_heads, sq, sk, head_dim, past_sk, scale, 1,
                   layer_window, mask_window, out);
}

/* reshape_to_bhsd / reshape_from_bhsd -- microsoft.rs:660-704. */
static void reshape_to_bhsd(const float* src, int b, int sq, int heads, int d, float* out) {
  for (int bi = 0; bi < b; ++bi)
    for (int si = 0; si < sq; ++si)
      for (int hi = 0; hi < heads; ++hi)
        for (int di = 0; di < d; ++di)
          out[(((size_t)bi * heads + hi) * sq + si) * d + di] =
              src[(((size_t)bi * sq + si) * heads + hi) * d + di];
}

static void reshape_from_bhsd(const float* src, int b, int heads, int sq, int d, float* out) {
  for (int bi = 0; bi < b; ++bi)
    for (int hi = 0; hi < heads; ++hi)
      for (int si = 0; si < sq; ++si)
        for (int di = 0; di < d; ++di)
          out[(((size_t)bi * sq + si) * heads + hi) * d + di] =
              src[(((size_t)bi * heads + hi) * sq + si) * d + di];
}

/* kv_copy_block -- microsoft.rs:736-757. */
static void kv_copy_block(float* dst, const float* src, int batch, int heads, int src_sk,
                          int total_sk, int d, int dst_start) {
  for (int bi = 0; bi < batch; ++bi)
    for (int hi = 0; hi < heads; ++hi)
      for (int si = 0; si < src_sk; ++si)
        memcpy(dst + (((size_t)bi * heads + hi) * total_sk + dst_start + si) * d,
               src + (((size_t)bi * heads + hi) * src_sk + si) * d, sizeof(float) * (size_t)d);
}

/* ------------------------------------------------------------------------
 * op_group_query_attention -- onnx-rt/src/ops/microsoft.rs:1082-1190 with
 * gqa_validate (:933-984), gqa_apply_rotary (:1004-1052), kv_concat
 * (:762-792). Always causal (:1156).
 * ---------------------------------------------------------------------- */
int sai_or_gqa(const float* query, const float* key, const float* value, int b, int sq,
               int q_hidden, int kv_hidden, const float* past_k, const float* past_v,
               int past_sk, const float* cos_cache, const float* sin_cache, int cache_rows,
               int cache_cols, int num_heads, int kv_num_heads, int has_scale, float scale_attr,
               int local_window_size, int do_rotary, int rotary_interleaved, float* attn_out,
               float* present_k, float* present_v) {
  if (local_window_size != -1) return ERR_INVALID_ATTRIBUTE;
  if (num_heads <= 0 || kv_num_heads <= 0) return ERR_INVALID_ATTRIBUTE;
  if (num_heads % kv_num_heads != 0) return ERR_INVALID_ATTRIBUTE;
  if (q_hidden % num_heads != 0) return ERR_SHAPE_MISMATCH;
  if (kv_hidden % kv_num_heads != 0) return ERR_SHAPE_MISMATCH;
  int head_dim = q_hidden / num_heads;
  if (kv_hidden / kv_num_heads != head_dim) return ERR_SHAPE_MISMATCH;
  if (past_sk != 0 && (past_k == NULL || past_v == NULL)) return ERR_SHAPE_MISMATCH;

  size_t nq = (size_t)b * num_heads * sq * head_dim;
  size_t nk = (size_t)b * kv_num_heads * sq * head_dim;
  float* q_bhsd = (float*)malloc(sizeof(float) * (nq ? nq : 1));
  float* k_bhsd = (float*)malloc(sizeof(float) * (nk ? nk : 1));
  float* v_bhsd = (float*)malloc(sizeof(float) * (nk ? nk : 1));
  reshape_to_bhsd(query, b, sq, num_heads, head_dim, q_bhsd);
  reshape_to_bhsd(key, b, sq, kv_num_heads, head_dim, k_bhsd);
  reshape_to_bhsd(value, b, sq, kv_num_heads, head_dim, v_bhsd);
  int rc = OK;
  if (do_rotary) {
    if (cos_cache == NULL || sin_cache == NULL) {
      rc = ERR_SHAPE_MISMATCH;
      goto done;
    }
    int64_t* pos = (int64_t*)malloc(sizeof(int64_t) * (size_t)(sq ? sq : 1));
    for (int i = 0; i < sq; ++i) pos[i] = (int64_t)past_sk + i;
    rc = sai_or_apply_rope(q_bhsd, b, num_heads, sq, head_dim, cos_cache, sin_cache, cache_rows,
                           cache_cols, pos, sq, rotary_interleaved, head_dim);
    if (rc == OK)
      rc = sai_or_apply_rope(k_bhsd, b, kv_num_heads, sq, head_dim, cos_cache, sin_cache,
                             cache_rows, cache_cols, pos, sq, rotary_interleaved, head_dim);
    free(pos);
    if (rc != OK) goto done;
  }
  {
    int total = past_sk + sq;
    if (past_k) kv_copy_block(present_k, past_k, b, kv_num_heads, past_sk, total, head_dim, 0);
    kv_copy_block(present_k, k_bhsd, b, kv_num_heads, sq, total, head_dim, past_sk);
    if (past_v) kv_copy_block(present_v, past_v, b, kv_num_heads, past_sk, total, head_dim, 0);
    kv_copy_block(present_v, v_bhsd, b, kv_num_heads, sq, total, head_dim, past_sk);
    float scale = has_scale ? scale_attr : sai_or_default_scale(head_dim);
    float* out_bhsd = (float*)malloc(sizeof(float) * (nq ? nq : 1));
    rc = sai_or_sdpa(q_bhsd, present_k, present_v, b, num_heads, kv_num_heads, sq, total,
                     head_dim, past_sk, scale, 1, out_bhsd);
    if (rc == OK) reshape_from_bhsd(out_bhsd, b, num_heads, sq, head_dim, attn_out);
    free(out_bhsd);
  }
done:
  free(q_bhsd);
  free(k_bhsd);
  free(v_bhsd);
  return rc;
}

/* ------------------------------------------------------------------------
 * Composed KV quantisation spec. The reference has no per-token-per-head or
 * group-32 KV quantiser; these compose its primitives:
 *  int8: amax over the row; s = amax/127 (1.0 when amax == 0, the range==0
 *        convention of kv_compression.rs:237-241); code =
 *        clamp(round_half_even(x/s) as i32 + 0, -128, 127)
 *        (QuantizeLinear, ops/quantized.rs:139-141); dequant q as f32 * s
 *        (DequantizeLinear, ops/quantized.rs:176-179).
 *  int4: per group of 32 along D, min/max quantiser of PolarQuantizer::encode
 *        (kv_compression.rs:223-253) with levels = 15, scale and zero point
 *        stored as IEEE binary16 and used as stored; codes packed LSB-first
 *        (kv_compression.rs:294-312); dequant q * s + z (kv_compression.rs:277-280).
 * ---------------------------------------------------------------------- */
void sai_or_quant_int8_row(const float* x, int d, int8_t* codes, float* scale) {
  float amax = 0.0f;
  for (int i = 0; i < d; ++i) {
    float a = fabsf(x[i]);
    if (a > amax) amax = a;
  }
  float s = (amax > 0.0f) ? amax / 127.0f : 1.0f;
  for (int i = 0; i < d; ++i) {
    int32_t q = sai_or_sat_i32(sai_or_round_half_even(x[i] / s));
    if (q < -128) q = -128;
    if (q > 127) q = 127;
    codes[i] = (int8_t)q;
  }
  *scale = s;
}

void sai_or_dequant_int8_row(const int8_t* codes, float scale, int d, float* out) {
  for (int i = 0; i < d; ++i) out[i] = (float)codes[i] * scale;
}

void sai_or_quant_int4_row(const float* x, int d, uint8_t* packed, uint16_t* scale_f16,
                           uint16_t* zero_f16) {
  uint32_t q[32];
  for (int g = 0; g < d / 32; ++g) {
    const float* xg = x + g * 32;
    float mn = INFINITY, mx = -INFINITY;
    for (int i = 0; i < 32; ++i) {
      if (xg[i] < mn) mn = xg[i];
      if (xg[i] > mx) mx = xg[i];
    }
    float range = mx - mn;
    float scale = (range > 0.0f) ? range / 15.0f : 1.0f;
    uint16_t s16 = sai_or_f32_to_f16(scale);
    uint16_t z16 = sai_or_f32_to_f16(mn);
    float sf = sai_or_f16_to_f32(s16);
    float zf = sai_or_f16_to_f32(z16);
    for (int i = 0; i < 32; ++i) {
      uint32_t v = (sf > 0.0f) ? sai_or_sat_u32(sai_or_round_f32_kv((xg[i] - zf) / sf)) : 0u;
      q[i] = v < 15u ? v : 15u;
    }
    sai_or_pack_bits(q, 32, 4, packed + g * 16);
    scale_f16[g] = s16;
    zero_f16[g] = z16;
  }
}

void sai_or_dequant_int4_row(const uint8_t* packed, const uint16_t* scale_f16,
                             const uint16_t* zero_f16, int d, float* out) {
  uint32_t q[32];
  for (int g = 0; g < d / 32; ++g) {
    sai_or_unpack_bits(packed + g * 16, 16, 32, 4, q);
    float sf = sai_or_f16_to_f32(scale_f16[g]);
    float zf = sai_or_f16_to_f32(zero_f16[g]);
    for (int i = 0; i < 32; ++i) out[g * 32 + i] = (float)q[i] * sf + zf;
  }
}

/* ------------------------------------------------------------------------
 * Quantised-cache step: KV append (RoPE K, then quantise) and attention over
 * the dequantised cache. RoPE follows gqa_apply_rotary (microsoft.rs:1004-1052,
 * positions past_sk + i); attention follows op_group_query_attention
 * (:1082-1190) with the present K/V taken from the dequantised cache.
 * ---------------------------------------------------------------------- */
int sai_or_kv_append(const float* k_new, const float* v_new, int b, int s_new, int kv_heads,
                     int head_dim, const int32_t* start_pos, const float* cos_cache,
                     const float* sin_cache, int cache_rows, int do_rotary, int interleaved,
                     int quant, int t_cap, void* k_codes, void* v_codes, float* k_scale,
                     float* v_scale, uint16_t* k_sz, uint16_t* v_sz) {
  if (quant != 1 && quant != 2) return ERR_INVALID_ATTRIBUTE;
  if (quant == 2 && head_dim % 32 != 0) return ERR_SHAPE_MISMATCH;
  if (do_rotary && (cos_cache == NULL || sin_cache == NULL)) return ERR_SHAPE_MISMATCH;
  float* row = (float*)malloc(sizeof(float) * (size_t)head_dim);
  int ng = head_dim / 32;
  for (int bi = 0; bi < b; ++bi) {
    for (int s = 0; s < s_new; ++s) {
      int t = start_pos[bi] + s;
      if (t < 0 || t >= t_cap) {
        free(row);
        return ERR_SHAPE_MISMATCH;
      }
      for (int h = 0; h < kv_heads; ++h) {
        size_t src = (((size_t)bi * s_new + s) * kv_heads + h) * head_dim;
        size_t tok = ((size_t)bi * kv_heads + h) * t_cap + t;
        for (int which = 0; which < 2; ++which) {
          const float* in = which == 0 ? k_new : v_new;
          memcpy(row, in + src, sizeof(float) * (size_t)head_dim);
          if (which == 0 && do_rotary) {
            int64_t pos = t;
            int rc = sai_or_apply_rope(row, 1, 1, 1, head_dim, cos_cache, sin_cache, cache_rows,
                                       head_dim / 2, &pos, 1, interleaved, head_dim);
            if (rc != OK) {
              free(row);
              return rc;
            }
          }
          if (quant == 1) {
            int8_t* codes = (int8_t*)(which == 0 ? k_codes : v_codes);
            float* sc = which == 0 ? k_scale : v_scale;
            sai_or_quant_int8_row(row, head_dim, codes + tok * head_dim, sc + tok);
          } else {
            uint8_t* codes = (uint8_t*)(which == 0 ? k_codes : v_codes);
            uint16_t* sz = which == 0 ? k_sz : v_sz;
            /* sz layout [.., T, ng, 2]: scale then zero per group */
            uint16_t sc16[8], z16[8];
            sai_or_quant_int4_row(row, head_dim, codes + tok * (head_dim / 2), sc16, z16);
            for (int g = 0; g < ng; ++g) {
              sz[(tok * ng + g) * 2 + 0] = sc16[g];
              sz[(tok * ng + g) * 2 + 1] = z16[g];
            }
          }
        }
      }
    }
  }
  free(row);
  return OK;
}

int sai_or_kv_dequant(int b, int kv_heads, int head_dim, int quant, int t_cap,
                      const int32_t* seq_len, const void* k_codes, const void* v_codes,
                      const float* k_scale, const float* v_scale, const uint16_t* k_sz,
                      const uint16_t* v_sz, float* k_out, float* v_out) {
  if (quant != 1 && quant != 2) return ERR_INVALID_ATTRIBUTE;
  int ng = head_dim / 32;
  for (int bi = 0; bi < b; ++bi) {
    if (seq_len[bi] < 0 || seq_len[bi] > t_cap) return ERR_SHAPE_MISMATCH;
    for (int h = 0; h < kv_heads; ++h) {
      for (int t = 0; t < seq_len[bi]; ++t) {
        size_t tok = ((size_t)bi * kv_heads + h) * t_cap + t;
        if (quant == 1) {
          sai_or_dequant_int8_row((const int8_t*)k_codes + tok * head_dim, k_scale[tok], head_dim,
                                  k_out + tok * head_dim);
          sai_or_dequant_int8_row((const int8_t*)v_codes + tok * head_dim, v_scale[tok], head_dim,
                                  v_out + tok * head_dim);
        } else {
          uint16_t ks[8], kz[8], vs[8], vz[8];
          for (int g = 0; g < ng; ++g) {
            ks[g] = k_sz[(tok * ng + g) * 2 + 0];
            kz[g] = k_sz[(tok * ng + g) * 2 + 1];
            vs[g] = v_sz[(tok * ng + g) * 2 + 0];
            vz[g] = v_sz[(tok * ng + g) * 2 + 1];
          }
          sai_or_dequant_int4_row((const uint8_t*)k_codes + tok * (head_dim / 2), ks, kz,
                                  head_dim, k_out + tok * head_dim);
          sai_or_dequant_int4_row((const uint8_t*)v_codes + tok * (head_dim / 2), vs, vz,
                                  head_dim, v_out + tok * head_dim);
        }
      }
    }
  }
  return OK;
}

int sai_or_gqa_cached(const float* query, int b, int sq, int num_heads, int kv_heads,
                      int head_dim, const int32_t* seq_len, int t_cap, const float* k_deq,
                      const float* v_deq, const float* cos_cache, const float* sin_cache,
                      int cache_rows, int do_rotary, int interleaved, int has_scale,
                      float scale_attr, float* out) {
  return sai_or_gqa_cached_window(query, b, sq, num_heads, kv_heads, head_dim, seq_len, t_cap,
                                  k_deq, v_deq, cos_cache, sin_cache, cache_rows, do_rotary,
                                  interleaved, has_scale, scale_attr, 0, 0, out);
}

int sai_or_gqa_cached_window(const float* query, int b, int sq, int num_heads, int kv_heads,
                             int head_dim, const int32_t* seq_len, int t_cap, const float* k_deq,
                             const float* v_deq, const float* cos_cache, const float* sin_cache,
                             int cache_rows, int do_rotary, int interleaved, int has_scale,
                             float scale_attr, int layer_window, int mask_window, float* out) {
  if (num_heads <= 0 || kv_heads <= 0 || num_heads % kv_heads != 0) return ERR_INVALID_ATTRIBUTE;
  if (do_rotary && (cos_cache == NULL || sin_cache == NULL)) return ERR_SHAPE_MISMATCH;
  float scale = has_scale ? scale_attr : sai_or_default_scale(head_dim);
  size_t qrow = (size_t)num_heads * head_dim;
  float* q_bhsd = (float*)malloc(sizeof(float) * qrow * (size_t)sq);
  float* o_bhsd = (float*)malloc(sizeof(float) * qrow * (size_t)sq);
  int rc = OK;
  for (int bi = 0; bi < b && rc == OK; ++bi) {
    int total = seq_len[bi];
    int past = total - sq;
    if (past < 0 || total > t_cap) {
      rc = ERR_SHAPE_MISMATCH;
      break;
    }
    reshape_to_bhsd(query + (size_t)bi * sq * qrow, 1, sq, num_heads, head_dim, q_bhsd);
    if (do_rotary) {
      int64_t* pos = (int64_t*)malloc(sizeof(int64_t) * (size_t)(sq ? sq : 1));
      for (int i = 0; i < sq; ++i) pos[i] = (int64_t)past + i;
      rc = sai_or_apply_rope(q_bhsd, 1, num_heads, sq, head_dim, cos_cache, sin_cache,
                             cache_rows, head_dim / 2, pos, sq, interleaved, head_dim);
      free(pos);
      if (rc != OK) break;
    }
    /* present K/V for this sequence: copy out of the dequantised cache
     * (the kv_concat copy of microsoft.rs:762-792). */
    size_t n = (size_t)kv_heads * total * head_dim;
    float* kf = (float*)malloc(sizeof(float) * (n ? n : 1));
    float* vf = (float*)malloc(sizeof(float) * (n ? n : 1));
    for (int h = 0; h < kv_heads; ++h) {
      size_t src = (((size_t)bi * kv_heads + h) * t_cap) * head_dim;
      memcpy(kf + (size_t)h * total * head_dim, k_deq + src, sizeof(float) * (size_t)total * head_dim);
      memcpy(vf + (size_t)h * total * head_dim, v_deq + src, sizeof(float) * (size_t)total * head_dim);
    }
    rc = sdpa_impl(q_bhsd, kf, vf, 1, num_heads, kv_heads, sq, total, head_dim, past, scale, 1,
                   layer_window, mask_window, o_bhsd);
    free(kf);
    free(vf);
    if (rc == OK) reshape_from_bhsd(o_bhsd, 1, num_heads, sq, head_dim, out + (size_t)bi * sq * qrow);
  }
  free(q_bhsd);
  free(o_bhsd);
  return rc;
}

/* ------------------------------------------------------------------------ */
static inline int32_t code_i8(float r) {
  int32_t q = sai_or_sat_i32(r);
  if (q < -128) q = -128;
  if (q > 127) q = 127;
  return q;
}

uint64_t sai_or_check_rhe_vs_rint(uint64_t lo, uint64_t hi) {
  uint64_t bad = 0;
  for (uint64_t u = lo; u < (uint64_t)hi; ++u) {
    float x = u2f((uint32_t)u);
    if (code_i8(sai_or_round_half_even(x)) != code_i8(rintf(x))) ++bad;
  }
  return bad;
}

/* ------------------------------------------------------------------------
 * TurboQuant compressed KV (onnx-rt/src/kv_compression.rs), restated:
 * Xorshift64 (:44-67), wht_butterfly_normalize (:81-110), apply_signs
 * (:113-118), wht_with_signs / inverse_wht_with_signs (:124-140),
 * PolarQuantizer::new / encode / decode (:197-291), QJLResidualEncoder
 * encode / correction (:365-419), CompressedKVCache seeds (:766-790).
 * ---------------------------------------------------------------------- */
static uint64_t tq_xorshift_next(uint64_t* st) {
  uint64_t x = *st;
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  *st = x;
  return x;
}

void sai_or_tq_signs(uint64_t seed, int dim, int8_t* signs) {
  uint64_t st = seed ? seed : 0x5EEDDEADBEEFCAFEull;
  for (int i = 0; i < dim; ++i) signs[i] = (tq_xorshift_next(&st) & 1u) == 0 ? 1 : -1;
}

uint64_t sai_or_tq_head_seed(uint64_t seed, int layer, int num_kv_heads, int head) {
  return seed * 0x9E3779B97F4A7C15ull + (uint64_t)((size_t)layer * num_kv_heads + head);
}

static void tq_butterfly_normalize(float* x, int n) {
  for (int h = 1; h < n; h *= 2)
    for (int i = 0; i < n; i += 2 * h)
      for (int j = i; j < i + h; ++j) {
        float a = x[j], b = x[j + h];
        x[j] = a + b;
        x[j + h] = a - b;
      }
  float scale = 1.0f / sai_or_sqrt_approx((float)n);
  for (int i = 0; i < n; ++i) x[i] *= scale;
}

void sai_or_wht_with_signs(float* x, const int8_t* signs, int n) {
  for (int i = 0; i < n; ++i) x[i] *= (float)signs[i];
  tq_butterfly_normalize(x, n);
}

void sai_or_inverse_wht_with_signs(float* x, const int8_t* signs, int n) {
  tq_butterfly_normalize(x, n);
  for (int i = 0; i < n; ++i) x[i] *= (float)signs[i];
}

int sai_or_tq_encode(const float* input, int dim, int bits, const int8_t* signs, uint8_t* packed,
                     float* scale_out, float* zero_out, float* min_out, float* max_out) {
  if (dim <= 0 || (dim & (dim - 1)) != 0) return ERR_INVALID_ATTRIBUTE;
  if (bits != 3 && bits != 4 && bits != 8) return ERR_INVALID_ATTRIBUTE;
  float* rot = (float*)malloc(sizeof(float) * (size_t)dim);
  uint32_t* q = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)dim);
  memcpy(rot, input, sizeof(float) * (size_t)dim);
  sai_or_wht_with_signs(rot, signs, dim);
  float mn = INFINITY, mx = -INFINITY;
  for (int i = 0; i < dim; ++i) {
    if (rot[i] < mn) mn = rot[i];
    if (rot[i] > mx) mx = rot[i];
  }
  uint32_t levels = (1u << bits) - 1u;
  float range = mx - mn;
  float scale = range > 0.0f ? range / (float)levels : 1.0f;
  float zero = mn;
  for (int i = 0; i < dim; ++i) {
    uint32_t v = scale > 0.0f ? sai_or_sat_u32(sai_or_round_f32_kv((rot[i] - zero) / scale)) : 0u;
    q[i] = v < levels ? v : levels;
  }
  sai_or_pack_bits(q, (size_t)dim, bits, packed);
  *scale_out = scale;
  *zero_out = zero;
  if (min_out) *min_out = mn;
  if (max_out) *max_out = mx;
  free(rot);
  free(q);
  return OK;
}

void sai_or_tq_decode(const uint8_t* packed, int dim, int bits, float scale, float zero,
                      const int8_t* signs, float* out) {
  uint32_t* q = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)dim);
  sai_or_unpack_bits(packed, ((size_t)dim * bits + 7) / 8, (size_t)dim, bits, q);
  for (int i = 0; i < dim; ++i) out[i] = (float)q[i] * scale + zero;
  sai_or_inverse_wht_with_signs(out, signs, dim);
  free(q);
}

void sai_or_qjl_encode(const float* original, const float* approx, int dim, uint64_t* sign_bits,
                       float* c_out) {
  int words = (dim + 63) / 64;
  for (int w = 0; w < words; ++w) sign_bits[w] = 0;
  float sum = 0.0f;
  for (int i = 0; i < dim; ++i) {
    float r = original[i] - approx[i];
    sum += fabsf(r);
    if (r >= 0.0f) sign_bits[i / 64] |= 1ull << (i % 64);
  }
  *c_out = dim > 0 ? sum / (float)dim : 0.0f;
}

float sai_or_qjl_correction(const uint64_t* a_bits, float a_c, const uint64_t* b_bits, float b_c,
                            int dim) {
  if (dim == 0) return 0.0f;
  uint32_t pop = 0;
  for (int w = 0; w < (dim + 63) / 64; ++w) pop += (uint32_t)__builtin_popcountll(a_bits[w] ^ b_bits[w]);
  float sign_inner = (float)dim - 2.0f * (float)pop;
  return a_c * b_c * sign_inner / (float)dim;
}

/* CompressedKVCache::write_kv for one (layer, head) row (kv_compression.rs:
 * 814-860, low-rank K off): codes, scale, zero and, with qjl, the residual's
 * sign bits and mean |r| of the decoded row. */
int sai_or_tq_write_row(const float* x, int dim, int bits, const int8_t* signs, int qjl,
                        uint8_t* packed, float* scale, float* zero, uint64_t* sign_bits,
                        float* c) {
  int rc = sai_or_tq_encode(x, dim, bits, signs, packed, scale, zero, NULL, NULL);
  if (rc != OK || !qjl) return rc;
  float* approx = (float*)malloc(sizeof(float) * (size_t)dim);
  sai_or_tq_decode(packed, dim, bits, *scale, *zero, signs, approx);
  sai_or_qjl_encode(x, approx, dim, sign_bits, c);
  free(approx);
  return OK;
}

/* Decode attention over one (sequence, kv head) of a TurboQuant cache, the
 * read path of docs/kv-compression-design.md section 9 with the module's
 * inner-product estimator (kv_compression.rs:1254-1288): for each of the G
 * query heads, q is encoded with the head's quantizer; the logit of row t
 * is <decode(q), decode(k_t)> + (qjl ? correction(res(q), res(k_t)) : 0);
 * weights = softmax(scale * logits) as the SDPA softmax computes it
 * (max-subtracted expf_approx, microsoft.rs:270-299); out = sum_t w_t
 * decode(v_t). Row t's K/V: packed codes at k_codes + t*code_bytes, per-row
 * scale/zero/c arrays, sign words at k_signs + t*words. */
int sai_or_tq_attend(const float* q, int G, int dim, int bits, int qjl, const int8_t* signs,
                     int rows, const uint8_t* k_codes, const float* k_scale, const float* k_zero,
                     const uint64_t* k_signs, const float* k_c, const uint8_t* v_codes,
                     const float* v_scale, const float* v_zero, float scale, float* out) {
  int code_bytes = (dim * bits + 7) / 8, words = (dim + 63) / 64;
  float* qd = (float*)malloc(sizeof(float) * (size_t)dim);
  float* kd = (float*)malloc(sizeof(float) * (size_t)dim);
  float* logits = (float*)malloc(sizeof(float) * (size_t)(rows ? rows : 1));
  uint8_t* qp = (uint8_t*)malloc((size_t)code_bytes);
  uint64_t* qs = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)words);
  int rc = OK;
  for (int h = 0; h < G && rc == OK; ++h) {
    const float* qh = q + (size_t)h * dim;
    float qsc, qz, qc = 0.0f;
    rc = sai_or_tq_write_row(qh, dim, bits, signs, qjl, qp, &qsc, &qz, qs, &qc);
    if (rc != OK) break;
    sai_or_tq_decode(qp, dim, bits, qsc, qz, signs, qd);
    float mx = -INFINITY;
    for (int t = 0; t < rows; ++t) {
      sai_or_tq_decode(k_codes + (size_t)t * code_bytes, dim, bits, k_scale[t], k_zero[t], signs, kd);
      float dot = 0.0f;
      for (int i = 0; i < dim; ++i) dot += qd[i] * kd[i];
      if (qjl) dot += sai_or_qjl_correction(qs, qc, k_signs + (size_t)t * words, k_c[t], dim);
      logits[t] = dot * scale;
      if (logits[t] > mx) mx = logits[t];
    }
    float denom = 0.0f;
    for (int t = 0; t < rows; ++t) {
      logits[t] = sai_or_expf_approx(logits[t] - mx);
      denom += logits[t];
    }
    float* o = out + (size_t)h * dim;
    for (int i = 0; i < dim; ++i) o[i] = 0.0f;
    if (rows == 0 || !(denom > 0.0f)) continue;
    float inv = 1.0f / denom;
    for (int t = 0; t < rows; ++t) {
      sai_or_tq_decode(v_codes + (size_t)t * code_bytes, dim, bits, v_scale[t], v_zero[t], signs, kd);
      float w = logits[t] * inv;
      for (int i = 0; i < dim; ++i) o[i] += w * kd[i];
    }
  }
  free(qd);
  free(kd);
  free(logits);
  free(qp);
  free(qs);
  return rc;
}

/* The design's attention_logits (docs/kv-compression-design.md section 9,
 * step 4) with the module's estimator (kv_compression.rs:1254-1288): for
 * each of the G query heads, q is encoded with the head's quantizer and
 * logits[h][t] = <decode(q), decode(k_t)> + (qjl ? correction : 0), dot in
 * dim order. Unscaled. */
int sai_or_tq_attention_logits(const float* q, int G, int dim, int bits, int qjl,
                               const int8_t* signs, int rows, const uint8_t* k_codes,
                               const float* k_scale, const float* k_zero, const uint64_t* k_signs,
                               const float* k_c, float* logits) {
  int code_bytes = (dim * bits + 7) / 8, words = (dim + 63) / 64;
  float* qd = (float*)malloc(sizeof(float) * (size_t)dim);
  float* kd = (float*)malloc(sizeof(float) * (size_t)dim);
  uint8_t* qp = (uint8_t*)malloc((size_t)code_bytes);
  uint64_t* qs = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)words);
  int rc = OK;
  for (int h = 0; h < G && rc == OK; ++h) {
    float qsc, qz, qc = 0.0f;
    rc = sai_or_tq_write_row(q + (size_t)h * dim, dim, bits, signs, qjl, qp, &qsc, &qz, qs, &qc);
    if (rc != OK) break;
    sai_or_tq_decode(qp, dim, bits, qsc, qz, signs, qd);
    for (int t = 0; t < rows; ++t) {
      sai_or_tq_decode(k_codes + (size_t)t * code_bytes, dim, bits, k_scale[t], k_zero[t], signs, kd);
      float dot = 0.0f;
      for (int i = 0; i < dim; ++i) dot += qd[i] * kd[i];
      if (qjl) dot += sai_or_qjl_correction(qs, qc, k_signs + (size_t)t * words, k_c[t], dim);
      logits[(size_t)h * rows + t] = dot;
    }
  }
  free(qd);
  free(kd);
  free(qp);
  free(qs);
  return rc;
}

/* The design's weighted_value_sum (section 9, step 6): out[h] = sum_t
 * weights[h][t] * decode(v_t), rows in order, not normalised. */
void sai_or_tq_weighted_value_sum(const float* weights, int G, int dim, int bits,
                                  const int8_t* signs, int rows, const uint8_t* v_codes,
                                  const float* v_scale, const float* v_zero, float* out) {
  int code_bytes = (dim * bits + 7) / 8;
  float* vd = (float*)malloc(sizeof(float) * (size_t)dim);
  for (int i = 0; i < G * dim; ++i) out[i] = 0.0f;
  for (int t = 0; t < rows; ++t) {
    sai_or_tq_decode(v_codes + (size_t)t * code_bytes, dim, bits, v_scale[t], v_zero[t], signs, vd);
    for (int h = 0; h < G; ++h) {
      float w = weights[(size_t)h * rows + t];
      for (int i = 0; i < dim; ++i) out[(size_t)h * dim + i] += w * vd[i];
    }
  }
  free(vd);
}

/* --- LowRankKeyDecomposer (kv_compression.rs:420-690) ------------------- */

/* norm_vec (:674-680): sum of squares in index order, then sqrt_approx. */
static float lr_norm(const float* v, int n) {
  float s = 0.0f;
  for (int i = 0; i < n; ++i) s += v[i] * v[i];
  return sai_or_sqrt_approx(s);
}

/* normalize_vec (:683-690): divided by the norm when it exceeds 1e-30. */
static void lr_normalize(float* v, int n) {
  float nv = lr_norm(v, n);
  if (nv > 1e-30f)
    for (int i = 0; i < n; ++i) v[i] /= nv;
}

/* power_iteration_svd (:583-671) on a (m x n, row-major; deflated in place):
 * per component r, v starts at +-1 ((j + r) even: +1) normalised, ten rounds
 * of u = A v, v = A^T u (rows accumulated in order), v normalised; then
 * u = A v, sigma = |u|; sigma < 1e-12 ends the loop (the remaining columns
 * stay zero); U_S[:, r] = (u / sigma) * sigma, Vt[r] = v; A -= sigma u v^T. */
static void lr_power_svd(float* a, int m, int n, int rank, float* u_s, float* vt) {
  float* v = (float*)malloc(sizeof(float) * (size_t)n);
  float* u = (float*)malloc(sizeof(float) * (size_t)m);
  for (int i = 0; i < m * rank; ++i) u_s[i] = 0.0f;
  for (int i = 0; i < rank * n; ++i) vt[i] = 0.0f;
  for (int r = 0; r < rank; ++r) {
    for (int j = 0; j < n; ++j) v[j] = (j + r) % 2 == 0 ? 1.0f : -1.0f;
    lr_normalize(v, n);
    for (int it = 0; it < 10; ++it) {
      for (int i = 0; i < m; ++i) {
        float dot = 0.0f;
        for (int j = 0; j < n; ++j) dot += a[(size_t)i * n + j] * v[j];
        u[i] = dot;
      }
      for (int j = 0; j < n; ++j) v[j] = 0.0f;
      for (int i = 0; i < m; ++i)
        for (int j = 0; j < n; ++j) v[j] += a[(size_t)i * n + j] * u[i];
      lr_normalize(v, n);
    }
    for (int i = 0; i < m; ++i) {
      float dot = 0.0f;
      for (int j = 0; j < n; ++j) dot += a[(size_t)i * n + j] * v[j];
      u[i] = dot;
    }
    float sigma = lr_norm(u, m);
    if (sigma < 1e-12f) break;
    for (int i = 0; i < m; ++i) u[i] /= sigma;
    for (int i = 0; i < m; ++i) u_s[(size_t)i * rank + r] = u[i] * sigma;
    for (int j = 0; j < n; ++j) vt[(size_t)r * n + j] = v[j];
    for (int i = 0; i < m; ++i)
      for (int j = 0; j < n; ++j) a[(size_t)i * n + j] -= sigma * u[i] * v[j];
  }
  free(v);
  free(u);
}

/* decompose (:470-498): rank 0 counts as 1 (new, :461-465); the kept rank is
 * min(rank, rows, cols), returned; u_s [rows][kept], vt [kept][cols]. An
 * empty matrix keeps the requested rank with no factors. */
int sai_or_lr_decompose(const float* k, int rows, int cols, int rank, float* u_s, float* vt) {
  if (rank <= 0) rank = 1;
  if (rows == 0 || cols == 0) return rank;
  int kept = rank < rows ? rank : rows;
  if (cols < kept) kept = cols;
  float* a = (float*)malloc(sizeof(float) * (size_t)rows * cols);
  memcpy(a, k, sizeof(float) * (size_t)rows * cols);
  lr_power_svd(a, rows, cols, kept, u_s, vt);
  free(a);
  return kept;
}

/* reconstruct (:502-523): out[i][j] = sum over r in order of
 * u_s[i][r] * vt[r][j], from 0.0. */
void sai_or_lr_reconstruct(const float* u_s, const float* vt, int rows, int cols, int rank,
                           float* out) {
  for (int i = 0; i < rows; ++i)
    for (int j = 0; j < cols; ++j) {
      float s = 0.0f;
      for (int r = 0; r < rank; ++r) s += u_s[(size_t)i * rank + r] * vt[(size_t)r * cols + j];
      out[(size_t)i * cols + j] = rank > 0 ? s : 0.0f;
    }
}

/* update (:529-561) and reorthogonalize (:564-577): appends the row's
 * coefficients new_row . Vt[r] (u_s holds room for one more row), counts the
 * write, and every 512th write with rows > rank rebuilds U_S Vt and
 * decomposes it again at min(rank, rows, cols). */
void sai_or_lr_update(float* u_s, float* vt, int* rows, int cols, int* rank, int* write_counter,
                      const float* new_row) {
  int rk = *rank;
  if (rk == 0 || cols == 0) {
    *rows += 1;
    return;
  }
  for (int r = 0; r < rk; ++r) {
    float dot = 0.0f;
    for (int c = 0; c < cols; ++c) dot += new_row[c] * vt[(size_t)r * cols + c];
    u_s[(size_t)(*rows) * rk + r] = dot;
  }
  *rows += 1;
  *write_counter += 1;
  if (*write_counter % 512 == 0 && *rows > rk) {
    int m = *rows;
    int kept = rk < m ? rk : m;
    if (cols < kept) kept = cols;
    float* a = (float*)malloc(sizeof(float) * (size_t)m * cols);
    sai_or_lr_reconstruct(u_s, vt, m, cols, rk, a);
    lr_power_svd(a, m, cols, kept, u_s, vt);
    free(a);
    *rank = kept;
    *write_counter = 0;
  }
}
