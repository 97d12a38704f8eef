/*
 * ffkv_oracle.h - CPU restatement of Firefly's paged KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the checker the HIP path is compared against and the CPU baseline that
 * bench.py times; nothing in the product library links, loads or calls it.  Only tests/, the smoke() check in
 * __graft_entry__.py and bench.py's cpu_baseline leg use it.
 *
 * Signatures mirror include/ffkv.h (same argument meaning, same dtype codes, same return codes) minus the
 * stream/workspace arguments, so a test can run both on identical inputs.
 */
#ifndef FFKV_ORACLE_H_
#define FFKV_ORACLE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Scalar conversions (exposed so tests can pin them against numpy / torch). */
uint16_t ffo_f32_to_bf16(float x);
float    ffo_bf16_to_f32(uint16_t h);
uint16_t ffo_f32_to_f16(float x);
float    ffo_f16_to_f32(uint16_t h);
uint8_t  ffo_f32_to_e4m3(float x);
float    ffo_e4m3_to_f32(uint8_t q);
/* int8 per-token quantization of n contiguous values: returns the scale, writes n codes. */
float ffo_quant_i8_row(const float* x, int n, int8_t* q);

/* Batch converters (n elements). */
void ffo_cvt_f32_to_bf16(const float* x, uint16_t* y, size_t n);
void ffo_cvt_f32_to_f16(const float* x, uint16_t* y, size_t n);
void ffo_cvt_f32_to_e4m3(const float* x, uint8_t* y, size_t n);
void ffo_cvt_e4m3_to_f32(const uint8_t* x, float* y, size_t n);
void ffo_cvt_bf16_to_f32(const uint16_t* x, float* y, size_t n);
void ffo_cvt_f16_to_f32(const uint16_t* x, float* y, size_t n);

/* Restatement of the append kernel (src/model/qwen_model.cu:21-47) with quantization; see ffkv_append. */
int ffo_append(const void* k_src, const void* v_src, int src_dtype, void* k_cache, void* v_cache, int cache_dtype,
               float* k_scale, float* v_scale, const int32_t* block_table, const int32_t* context_lens, int batch,
               int seq_len, int num_kv_heads, int head_dim, int block_size, int max_blocks, int num_blocks);

/* Causal prefill over the paged cache (queries at ctx + t, prefix included) or, with block_table == NULL, over
 * contiguous [batch, seq_len, Hkv, D] K/V (the reference's prefill branch); float64 closed form, out
 * [batch, seq_len, num_heads, head_dim]. */
int ffo_paged_prefill_f64(const void* q, int qo_dtype, const void* k_cache, const void* v_cache, int cache_dtype,
                          const float* k_scale, const float* v_scale, const int32_t* block_table,
                          const int32_t* context_lens, int batch, int seq_len, int num_heads, int num_kv_heads,
                          int head_dim, int max_blocks, int num_blocks, int max_context_len, float scale, double* out);

/* Rotary embedding in place of x [batch, seq_len, heads, head_dim] (src/kernels/rope.cu:22-137); see ffkv_rope. */
int ffo_rope(void* x, int dtype, const int32_t* context_lens, int batch, int seq_len, int heads, int head_dim,
             float theta);

/*
 * Restatement of paged_attention_kernel (src/kernels/attention.cu:291-447): per (sequence, query head), eight
 * interleaved token groups each run an online softmax in fp32, then the eight states are merged.  Output is
 * rounded to qo_dtype.  If out_f32 is non-NULL the fp32 value before rounding is stored there too
 * ([batch, num_heads, head_dim]).  threads <= 0 uses all host cores.
 */
int ffo_paged_decode(const void* q, void* out, int qo_dtype, const void* k_cache, const void* v_cache,
                     int cache_dtype, const float* k_scale, const float* v_scale, const int32_t* block_table,
                     const int32_t* context_lens, int batch, int num_heads, int num_kv_heads, int head_dim,
                     int block_size, int max_blocks, int num_blocks, int max_context_len, float scale,
                     float* out_f32, int threads);

/* Closed form in float64: softmax(scale * q.K^T) V over the gathered, dequantized tokens.  out is
 * [batch, num_heads, head_dim] double. */
int ffo_paged_decode_f64(const void* q, int qo_dtype, const void* k_cache, const void* v_cache, int cache_dtype,
                         const float* k_scale, const float* v_scale, const int32_t* block_table,
                         const int32_t* context_lens, int batch, int num_heads, int num_kv_heads, int head_dim,
                         int block_size, int max_blocks, int num_blocks, int max_context_len, float scale,
                         double* out);

/* Number of host threads ffo_paged_decode uses for threads <= 0. */
int ffo_default_threads(void);

#ifdef __cplusplus
}
#endif

#endif /* FFKV_ORACLE_H_ */
