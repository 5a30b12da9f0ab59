// C-ABI exports over the reference's own header-only implementation.
//
// TEST INFRASTRUCTURE ONLY.  This file contains no reference code: it
// #includes the reference headers where they lie (-I<reference>/include, see
// oracle/Makefile) and exports their functions unchanged so the restatement
// in attn_oracle.c can be checked against them, and so bench.py can time the
// reference's own CPU path as its cpu_baseline.  The built library goes to
// oracle/_ref/ (git-ignored).
#include <cstdint>
#include <cstring>
#include <stdexcept>

#include "molot/attn.h"
#include "molot/norm.h"
#include "molot/quant.h"
#include "molot/thread_pool.h"

extern "C" {

void* ref_pool_create(int nthreads) { return new molot::ThreadPool(nthreads); }
void ref_pool_destroy(void* p) { delete static_cast<molot::ThreadPool*>(p); }
int ref_pool_size(void* p) { return static_cast<molot::ThreadPool*>(p)->size(); }

// ThreadPool::parallel_for coverage probe (bench/bench.cc:59-66 style):
// writes 1 into seen[i] for every index the pool visits.
void ref_pool_cover(void* p, int64_t n, int32_t* seen) {
  static_cast<molot::ThreadPool*>(p)->parallel_for(n, [&](int, int64_t i) { seen[i] += 1; });
}

void ref_rope_inv_freq(float base, int d, float* out) { molot::rope_inv_freq(base, d, out); }

void ref_rope_apply(float* x, int d, int pos, const float* inv_freq) {
  molot::rope_apply(x, d, pos, inv_freq);
}

void ref_exp16(const float* in, float* out) {
  _mm512_storeu_ps(out, molot::exp_avx512_ps(_mm512_loadu_ps(in)));
}

float ref_dot(const float* a, const float* b, int n) { return molot::dot_fp32_avx512(a, b, n); }

uint16_t ref_fp32_to_bf16(float f) { return molot::fp32_to_bf16(f); }
float ref_bf16_to_fp32(uint16_t b) { return molot::bf16_to_fp32(b); }

void ref_attn_decode_head_win(const float* Q, const float* K, const float* V, float* out, int n,
                              int d, float scale, int pos_cur, int window) {
  molot::attn_decode_head_win(Q, K, V, out, n, d, scale, pos_cur, window);
}

void ref_attn_decode_head(const float* Q, const float* K, const float* V, float* out, int n,
                          int d, float scale) {
  molot::attn_decode_head(Q, K, V, out, n, d, scale);
}

void ref_attn_decode_gqa(const float* Q, const float* K, const float* V, float* O, int nq, int nkv,
                         int n, int d, float scale, void* pool) {
  molot::attn_decode_gqa(Q, K, V, O, nq, nkv, n, d, scale,
                         *static_cast<molot::ThreadPool*>(pool));
}

void ref_attn_decode_gqa_cache(const float* Q, const float* K, const float* V, float* O, int nq,
                               int nkv, int n, int qhd, float scale, int pos_cur, int window,
                               void* pool) {
  molot::attn_decode_gqa_cache(Q, K, V, O, nq, nkv, n, qhd, scale, pos_cur, window,
                               *static_cast<molot::ThreadPool*>(pool));
}

void ref_attn_decode_gqa_win(const float* Q, const float* K, const float* V, float* O, int nq,
                             int nkv, int n, int d, float scale, int pos_cur, int window,
                             void* pool) {
  molot::attn_decode_gqa_win(Q, K, V, O, nq, nkv, n, d, scale, pos_cur, window,
                             *static_cast<molot::ThreadPool*>(pool));
}

// The decode-attention block of Runner::forward_token (forward.h:556-591)
// for one layer with its own KV: rope q heads, rope k heads, append k/v at
// slot `slot` of the [cap][nkv*d] cache, attention over n = slot + 1.
// A NULL inv_freq is a layer without RoPE (an empty L.freq): forward.h:556
// and :566 then skip rope_apply.  Returns 0, or -1 where forward.h:570
// would throw "KV cache full".
int ref_decode_step(float* q, float* k, const float* v, float* Kc, float* Vc, float* O, int nq,
                    int nkv, int d, int slot, int cap, int pos, const float* inv_freq, float scale,
                    int window, void* pool) {
  if (inv_freq)  // forward.h:556, :566: no rotation for a layer without RoPE
    for (int hh = 0; hh < nq; ++hh) molot::rope_apply(q + (size_t)hh * d, d, pos, inv_freq);
  if (inv_freq)
    for (int hh = 0; hh < nkv; ++hh) molot::rope_apply(k + (size_t)hh * d, d, pos, inv_freq);
  if (slot >= cap) return -1;
  std::memcpy(Kc + (size_t)slot * nkv * d, k, (size_t)nkv * d * 4);
  std::memcpy(Vc + (size_t)slot * nkv * d, v, (size_t)nkv * d * 4);
  molot::attn_decode_gqa_cache(q, Kc, Vc, O, nq, nkv, slot + 1, d, scale, pos, window,
                               *static_cast<molot::ThreadPool*>(pool));
  return 0;
}

void ref_attn_prefill_gqa(const float* Qm, const float* K, const float* V, float* Om, int nq,
                          int nkv, int M, int N, int d, float scale, int pos0, int window,
                          void* pool) {
  molot::attn_prefill_gqa(Qm, K, V, Om, nq, nkv, M, N, d, scale, pos0, window,
                          *static_cast<molot::ThreadPool*>(pool));
}

// One layer's prefill in forward.h's order (forward.h:367-399): per token
// q heads RMS-normed with q_norm and rotated at pos0 + m, k heads normed
// with k_norm, v normed over its nkv*d values when v_norm, k rotated, k/v
// appended at slot slot0 + m; then attn_prefill_gqa over N = slot0 + M.
// NULL weights skip a norm (forward.h always has them; the shim lets tests
// isolate RoPE + append); a NULL inv_freq skips RoPE, as forward.h:373 and
// :381 do for a layer without it.  Returns -1 where forward.h:380 would throw.
int ref_prefill_step(float* Q, float* Kn, float* Vn, float* Kc, float* Vc, float* O, int nq,
                     int nkv, int d, int M, int slot0, int cap, int pos0, const float* q_norm,
                     const float* k_norm, int v_norm, float eps, const float* inv_freq,
                     float scale, int window, void* pool) {
  if (slot0 + M > cap) return -1;
  for (int mm = 0; mm < M; ++mm) {
    float* qq = Q + (size_t)mm * nq * d;
    float* kk = Kn + (size_t)mm * nkv * d;
    float* vv = Vn + (size_t)mm * nkv * d;
    for (int hh = 0; hh < nq; ++hh) {
      if (q_norm) molot::rmsnorm(qq + (size_t)hh * d, q_norm, qq + (size_t)hh * d, d, eps);
      if (inv_freq) molot::rope_apply(qq + (size_t)hh * d, d, pos0 + mm, inv_freq);  // :373
    }
    if (k_norm)
      for (int hh = 0; hh < nkv; ++hh)
        molot::rmsnorm(kk + (size_t)hh * d, k_norm, kk + (size_t)hh * d, d, eps);
    if (v_norm) molot::rmsnorm_plain(vv, vv, nkv * d, eps);
    if (inv_freq)  // forward.h:381
      for (int hh = 0; hh < nkv; ++hh)
        molot::rope_apply(kk + (size_t)hh * d, d, pos0 + mm, inv_freq);
    std::memcpy(Kc + (size_t)(slot0 + mm) * nkv * d, kk, (size_t)nkv * d * 4);
    std::memcpy(Vc + (size_t)(slot0 + mm) * nkv * d, vv, (size_t)nkv * d * 4);
  }
  molot::attn_prefill_gqa(Q, Kc, Vc, O, nq, nkv, M, slot0 + M, d, scale, pos0, window,
                          *static_cast<molot::ThreadPool*>(pool));
  return 0;
}

// quantize_q8_row (quant.h:34-50) on one row: scale, int8 values, and the
// per-32 block sums it also writes (ignored by the KV format).
void ref_quantize_q8_row(const float* x, int cols, float* scale, int8_t* q) {
  const int nblocks = (cols + 31) / 32;
  int32_t bsums[64];
  if (nblocks > 64) return;
  molot::quantize_q8_row(x, cols, nblocks, scale, q, bsums);
}

void ref_rmsnorm(const float* x, const float* w, float* y, int n, float eps) {
  molot::rmsnorm(x, w, y, n, eps);
}

void ref_rmsnorm_plain(const float* x, float* y, int n, float eps) {
  molot::rmsnorm_plain(x, y, n, eps);
}

// forward.h:554-591 with the layer's norms, in forward.h's order: q heads
// RMS-normed with q_norm (Runner::rms_per_head, forward.h:138-140) and
// rotated; k heads normed with k_norm, v normed over all its nkv*d values
// when v_norm (forward.h:562-563), k rotated; append; attention.  A NULL
// inv_freq skips both rotations (forward.h:556, :566).
int ref_decode_step_norm(float* q, float* k, float* v, float* Kc, float* Vc, float* O, int nq,
                         int nkv, int d, int slot, int cap, int pos, const float* q_norm,
                         const float* k_norm, int v_norm, float eps, const float* inv_freq,
                         float scale, int window, void* pool) {
  for (int hh = 0; hh < nq; ++hh)
    molot::rmsnorm(q + (size_t)hh * d, q_norm, q + (size_t)hh * d, d, eps);
  if (inv_freq)  // forward.h:556
    for (int hh = 0; hh < nq; ++hh) molot::rope_apply(q + (size_t)hh * d, d, pos, inv_freq);
  for (int hh = 0; hh < nkv; ++hh)
    molot::rmsnorm(k + (size_t)hh * d, k_norm, k + (size_t)hh * d, d, eps);
  if (v_norm) molot::rmsnorm_plain(v, v, nkv * d, eps);
  if (inv_freq)  // forward.h:566
    for (int hh = 0; hh < nkv; ++hh) molot::rope_apply(k + (size_t)hh * d, d, pos, inv_freq);
  if (slot >= cap) return -1;
  std::memcpy(Kc + (size_t)slot * nkv * d, k, (size_t)nkv * d * 4);
  std::memcpy(Vc + (size_t)slot * nkv * d, v, (size_t)nkv * d * 4);
  molot::attn_decode_gqa_cache(q, Kc, Vc, O, nq, nkv, slot + 1, d, scale, pos, window,
                               *static_cast<molot::ThreadPool*>(pool));
  return 0;
}

// A decode step of a layer without its own KV (L.has_kv false), in
// forward.h's order: q heads RMS-normed with q_norm (forward.h:554; NULL
// skips it) and rotated at pos when inv_freq is given (:556-558), then
// attn_decode_gqa_cache over the source layer's cache Kc/Vc and its n
// slots (:578-591).  Returns -1 where forward.h:580 would throw "shared KV
// empty" (n == 0).
int ref_decode_step_shared(float* q, const float* Kc, const float* Vc, float* O, int nq, int nkv,
                           int d, int n, int pos, const float* q_norm, float eps,
                           const float* inv_freq, float scale, int window, void* pool) {
  if (n == 0) return -1;
  if (q_norm)
    for (int hh = 0; hh < nq; ++hh)
      molot::rmsnorm(q + (size_t)hh * d, q_norm, q + (size_t)hh * d, d, eps);
  if (inv_freq)
    for (int hh = 0; hh < nq; ++hh) molot::rope_apply(q + (size_t)hh * d, d, pos, inv_freq);
  molot::attn_decode_gqa_cache(q, Kc, Vc, O, nq, nkv, n, d, scale, pos, window,
                               *static_cast<molot::ThreadPool*>(pool));
  return 0;
}

// The prefill of a layer without its own KV (forward.h:367-399 with
// L.has_kv false): per token m the q heads normed with q_norm (NULL: none)
// and rotated at pos0 + m when inv_freq is given (:370-375), nothing
// appended, then attn_prefill_gqa over the source cache's N slots (:394-398).
void ref_prefill_shared(float* Q, const float* Kc, const float* Vc, float* O, int nq, int nkv,
                        int d, int M, int N, int pos0, const float* q_norm, float eps,
                        const float* inv_freq, float scale, int window, void* pool) {
  for (int mm = 0; mm < M; ++mm) {
    float* qq = Q + (size_t)mm * nq * d;
    for (int hh = 0; hh < nq; ++hh) {
      if (q_norm) molot::rmsnorm(qq + (size_t)hh * d, q_norm, qq + (size_t)hh * d, d, eps);
      if (inv_freq) molot::rope_apply(qq + (size_t)hh * d, d, pos0 + mm, inv_freq);
    }
  }
  molot::attn_prefill_gqa(Q, Kc, Vc, O, nq, nkv, M, N, d, scale, pos0, window,
                          *static_cast<molot::ThreadPool*>(pool));
}

}  // extern "C"
