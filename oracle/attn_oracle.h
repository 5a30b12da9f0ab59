/* C API of the CPU oracle (attn_oracle.c) -- TEST INFRASTRUCTURE ONLY.
 * Only tests (and bench.py's cpu_baseline leg) may include or link this. */
#ifndef MOLOT_ORACLE_ATTN_ORACLE_H_
#define MOLOT_ORACLE_ATTN_ORACLE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_KV_F32 0
#define ORC_KV_BF16 1
#define ORC_KV_Q8 2

uint16_t orc_f32_to_bf16(float f);
void orc_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n);
void orc_rope_inv_freq(float base, int d, float* out);
void orc_rope_apply(float* x, int d, int pos, const float* inv_freq);
void orc_rope_apply_heads(float* x, int nheads, int d, int pos, const float* inv_freq);
void orc_vexp16(const float* in, float* out);
float orc_dot(const float* a, const float* b, int n);
void orc_rmsnorm(const float* x, const float* w, float* y, int n, float eps);
int orc_q8_row_bytes(int nkv, int d);
int64_t orc_q8_block_bytes(int nkv, int d, int page);
void orc_quantize_q8_row(const float* x, int d, int8_t* q, float* s);
void orc_q8_store_token(void* base, int64_t t, const float* x, int nkv, int d);
void orc_q8_store_tokens(void* base, int64_t n, const float* x, int nkv, int d);
void orc_attn_decode(const float* Q, const void* K, const void* V, float* O, int nq, int nkv,
                     int n, int d, float scale, int pos_cur, int window, int kv_dtype,
                     int64_t tok_stride, int64_t head_stride, int64_t block_stride,
                     const int32_t* block_table, int page, int nthreads);
void orc_attn_decode_gqa_cache(const float* Q, const float* K, const float* V, float* O, int nq,
                               int nkv, int n, int qhd, float scale, int pos_cur, int window,
                               int nthreads);
void orc_decode_step(float* q, float* k_new, const float* v_new, void* Kc, void* Vc, float* O,
                     int nq, int nkv, int d, int slot, int pos, const float* inv_freq,
                     float scale, int window, int kv_dtype, int nthreads);
void orc_decode_step_norm(float* q, float* k_new, const float* v_new, void* Kc, void* Vc,
                          float* O, int nq, int nkv, int d, int slot, int pos,
                          const float* q_norm, const float* k_norm, int v_norm, float eps,
                          const float* inv_freq, float scale, int window, int kv_dtype,
                          int nthreads);
void orc_prefill_q(float* q, int nq, int d, int M, int pos0, const float* q_norm, float eps,
                   const float* inv_freq);
void orc_decode_step_shared(float* q, const void* Kc, const void* Vc, float* O, int nq, int nkv,
                            int d, int n, int pos, const float* q_norm, float eps,
                            const float* inv_freq, float scale, int window, int kv_dtype,
                            int nthreads);
void orc_attn_prefill(const float* Qm, const void* K, const void* V, float* Om, int nq, int nkv,
                      int M, int N, int d, float scale, int pos0, int window, int kv_dtype,
                      int nthreads);
void orc_attn_decode_f64(const float* Q, const void* K, const void* V, double* O, int nq,
                         int nkv, int n, int d, double scale, int pos_cur, int window,
                         int kv_dtype, int64_t tok_stride, int64_t head_stride,
                         int64_t block_stride, const int32_t* block_table, int page,
                         int nthreads);

#ifdef __cplusplus
}
#endif

#endif
