/*
 * CPU oracle for the compressed-KV GroupQueryAttention path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: tests/, the smoke
 * entry and the CPU-baseline leg of bench.py load it. The product library
 * (smallaios_amd/libsai_hip.so) never links, loads or calls it.
 *
 * It restates, op for op, the reference's Rust CPU semantics
 * (SmallAIOS onnx-rt, workspace 0.2.1). Every function cites the file:line
 * it follows. Arithmetic is plain IEEE f32 without contraction
 * (built with -ffp-contract=off -fno-fast-math), matching Rust, which never
 * fuses multiply-add on its own.
 *
 * Layout conventions (all little-endian, row-major):
 *   Q   [B, Sq, Hq*D]   K/V new [B, Sq, Hkv*D]   (ORT "BSH")
 *   past/present K/V [B, Hkv, S, D]               (ORT "BHSD")
 *   int8 cache codes [B, Hkv, T, D] int8, scales [B, Hkv, T] f32
 *   int4 cache codes [B, Hkv, T, D/2] u8 (pack_bits LSB-first along D),
 *        scale/zero [B, Hkv, T, D/32] f16 bits
 *
 * Return codes of the int functions: 0 ok, -1 InvalidAttribute,
 * -2 ShapeMismatch (the reference's OpError variants, operators.rs:26-37).
 */
#ifndef SAI_ORACLE_H
#define SAI_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* --- scalar numerics --------------------------------------------------- */
float sai_or_expf_approx(float x);
float sai_or_sqrt_f32(float x);
float sai_or_sqrt_approx(float x);
float sai_or_round_half_even(float x);
float sai_or_round_f32_kv(float x);
int32_t sai_or_sat_i32(float x);
uint32_t sai_or_sat_u32(float x);
int64_t sai_or_sat_i64(float x);
uint16_t sai_or_f32_to_bf16(float x);
float sai_or_bf16_to_f32(uint16_t b);
uint16_t sai_or_f32_to_f16(float x);
float sai_or_f16_to_f32(uint16_t h);
void sai_or_f32_to_f16_array(const float* x, size_t n, uint16_t* out);
void sai_or_round_half_even_array(const float* x, size_t n, float* out);
void sai_or_expf_approx_array(const float* x, size_t n, float* out);
float sai_or_default_scale(int head_dim);

/* --- bit packing ------------------------------------------------------- */
void sai_or_pack_bits(const uint32_t* values, size_t n, int bits, uint8_t* out);
void sai_or_unpack_bits(const uint8_t* data, size_t nbytes, size_t count, int bits,
                        uint32_t* out);

/* --- RoPE tables of the Gemma loader (f32 approximations) -------------- */
float sai_or_ln_approx(float x);
float sai_or_exp_approx(float x);
float sai_or_floor_approx(float x);
float sai_or_sin_approx(float x);
float sai_or_cos_approx(float x);
/* precompute_rope_tables: bf16 bits, row-major [max_pos, half]. */
void sai_or_rope_tables_bf16(int max_pos, int half, float rope_theta, uint16_t* cos_out,
                             uint16_t* sin_out);

/* --- TurboQuant compressed KV (kv_compression.rs) ---------------------- */
void sai_or_tq_signs(uint64_t seed, int dim, int8_t* signs);
uint64_t sai_or_tq_head_seed(uint64_t seed, int layer, int num_kv_heads, int head);
void sai_or_wht_with_signs(float* x, const int8_t* signs, int n);
void sai_or_inverse_wht_with_signs(float* x, const int8_t* signs, int n);
int sai_or_tq_encode(const float* input, int dim, int bits, const int8_t* signs, uint8_t* packed,
                     float* scale_out, float* zero_out, float* min_out, float* max_out);
void sai_or_tq_decode(const uint8_t* packed, int dim, int bits, float scale, float zero,
                      const int8_t* signs, float* out);
void sai_or_qjl_encode(const float* original, const float* approx, int dim, uint64_t* sign_bits,
                       float* c_out);
float sai_or_qjl_correction(const uint64_t* a_bits, float a_c, const uint64_t* b_bits, float b_c,
                            int dim);
int sai_or_tq_write_row(const float* x, int dim, int bits, const int8_t* signs, int qjl,
                        uint8_t* packed, float* scale, float* zero, uint64_t* sign_bits,
                        float* c);
int sai_or_tq_attend(const float* q, int G, int dim, int bits, int qjl, const int8_t* signs,
                     int rows, const uint8_t* k_codes, const float* k_scale, const float* k_zero,
                     const uint64_t* k_signs, const float* k_c, const uint8_t* v_codes,
                     const float* v_scale, const float* v_zero, float scale, float* out);

/* --- RoPE / SDPA / GQA (f32 reference op) ------------------------------ */
int sai_or_apply_rope(float* x, int b, int heads, int sq, int head_dim, const float* cos_cache,
                      const float* sin_cache, int cache_rows, int cache_cols,
                      const int64_t* position_ids, int n_pos, int interleaved, int rotary_dim);

int sai_or_sdpa(const float* q, const float* k, const float* v, int batch, int num_q_heads,
                int num_kv_heads, int sq, int sk, int head_dim, int past_sk, float scale,
                int causal, float* out);
/* Causal SDPA with the reference's window rules (layer_window: last keys of a
 * sliding-window cache layer; mask_window: the GPU mask's window); <= 0 = off. */
int sai_or_sdpa_window(const float* q, const float* k, const float* v, int batch,
                       int num_q_heads, int num_kv_heads, int sq, int sk, int head_dim,
                       int past_sk, float scale, int layer_window, int mask_window, float* out);

/* op_group_query_attention. past_k/past_v may be NULL (past_sk must then be 0).
 * scale_attr: used when has_scale != 0. Outputs: attn [B,Sq,Hq*D],
 * present_k/present_v [B,Hkv,past_sk+Sq,D]. */
int sai_or_gqa(const float* query, const float* key, const float* value, int b, int sq,
               int q_hidden, int kv_hidden, const float* past_k, const float* past_v,
               int past_sk, const float* cos_cache, const float* sin_cache, int cache_rows,
               int cache_cols, int num_heads, int kv_num_heads, int has_scale, float scale_attr,
               int local_window_size, int do_rotary, int rotary_interleaved, float* attn_out,
               float* present_k, float* present_v);

/* --- composed KV quantisation spec ------------------------------------- */
void sai_or_quant_int8_row(const float* x, int d, int8_t* codes, float* scale);
void sai_or_dequant_int8_row(const int8_t* codes, float scale, int d, float* out);
void sai_or_quant_int4_row(const float* x, int d, uint8_t* packed, uint16_t* scale_f16,
                           uint16_t* zero_f16);
void sai_or_dequant_int4_row(const uint8_t* packed, const uint16_t* scale_f16,
                             const uint16_t* zero_f16, int d, float* out);

/* --- composed quantized-cache step (the oracle of the HIP path) --------- */
/* KV append: for every (b, s, kvh) row of the new K/V ([B,S_new,Hkv*D] f32),
 * apply RoPE to K at position start_pos[b]+s (when do_rotary), quantize K and V
 * with the chosen spec and write codes/params at token index start_pos[b]+s of
 * the logical cache (capacity t_cap tokens per (b, kvh)).
 * quant: 1 = int8 sym per (token, head), 2 = int4 asym per group of 32. */
int sai_or_kv_append(const float* k_new, const float* v_new, int b, int s_new, int kv_heads,
                     int head_dim, const int32_t* start_pos, const float* cos_cache,
                     const float* sin_cache, int cache_rows, int do_rotary, int interleaved,
                     int quant, int t_cap, void* k_codes, void* v_codes, float* k_scale,
                     float* v_scale, uint16_t* k_sz, uint16_t* v_sz);

/* Dequantise the first seq_len[b] tokens of every (b, kvh) into f32
 * [B, Hkv, t_cap, D] (rows beyond seq_len are left untouched). */
int sai_or_kv_dequant(int b, int kv_heads, int head_dim, int quant, int t_cap,
                      const int32_t* seq_len, const void* k_codes, const void* v_codes,
                      const float* k_scale, const float* v_scale, const uint16_t* k_sz,
                      const uint16_t* v_sz, float* k_out, float* v_out);

/* Attention over the dequantised cache (new tokens already appended):
 * query [B, Sq, Hq*D] f32 (pre-RoPE), seq_len[b] = total keys for batch b
 * (past + Sq). Q is rotated at positions seq_len[b]-Sq+i, then causal SDPA
 * with past_sk = seq_len[b]-Sq. Per-batch, because ragged batches have a
 * different past_sk per sequence. out [B, Sq, Hq*D] f32. */
int sai_or_gqa_cached(const float* query, int b, int sq, int num_heads, int kv_heads,
                      int head_dim, const int32_t* seq_len, int t_cap, const float* k_deq,
                      const float* v_deq, const float* cos_cache, const float* sin_cache,
                      int cache_rows, int do_rotary, int interleaved, int has_scale,
                      float scale_attr, float* out);
int sai_or_gqa_cached_window(const float* query, int b, int sq, int num_heads, int kv_heads,
                             int head_dim, const int32_t* seq_len, int t_cap, const float* k_deq,
                             const float* v_deq, const float* cos_cache, const float* sin_cache,
                             int cache_rows, int do_rotary, int interleaved, int has_scale,
                             float scale_attr, int layer_window, int mask_window, float* out);

/* Exhaustive check that the int8 code rule built on round_half_even equals
 * the same rule built on IEEE roundTiesToEven (rintf) for every f32 bit
 * pattern u in [lo, hi) (hi <= 2^32). Returns the number of mismatches. */
uint64_t sai_or_check_rhe_vs_rint(uint64_t lo, uint64_t hi);

int sai_or_tq_attention_logits(const float* q, int G, int dim, int bits, int qjl,
                               const int8_t* signs, int rows, const uint8_t* k_codes,
                               const float* k_scale, const float* k_zero, const uint64_t* k_signs,
                               const float* k_c, float* logits);
void sai_or_tq_weighted_value_sum(const float* weights, int G, int dim, int bits,
                                  const int8_t* signs, int rows, const uint8_t* v_codes,
                                  const float* v_scale, const float* v_zero, float* out);

/* LowRankKeyDecomposer (kv_compression.rs:451-671). */
int sai_or_lr_decompose(const float* k, int rows, int cols, int rank, float* u_s, float* vt);
void sai_or_lr_reconstruct(const float* u_s, const float* vt, int rows, int cols, int rank,
                           float* out);
void sai_or_lr_update(float* u_s, float* vt, int* rows, int cols, int* rank, int* write_counter,
                      const float* new_row);

#ifdef __cplusplus
}
#endif

#endif
