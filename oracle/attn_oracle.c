/*
 * CPU oracle for the fused RoPE + GQA decode-attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker (or the timed CPU port); the product path (molot_amd/) never calls
 * it and has no CPU fallback.
 *
 * Two independent formulations live here:
 *
 *  1. A restatement of the reference algorithm in plain C (fp32, same pass
 *     order as the reference):
 *       orc_rope_inv_freq   <- include/molot/attn.h:31-33
 *       orc_rope_apply      <- include/molot/attn.h:19-28  (NEOX half-split)
 *       orc_vexp16          <- include/molot/norm.h:35-47  (clamp, Taylor-5, 2^k)
 *       orc_dot             <- include/molot/gemm.h:17-28  (16 lane accumulators)
 *       orc_attn_decode     <- include/molot/attn.h:125-177 (3 passes: scores,
 *                              vector exp + den, normalised PV), generalised
 *                              to strided / bf16 / paged K,V so the same
 *                              algorithm covers attn.h:57-120 and :178-187.
 *       orc_decode_step     <- include/molot/forward.h:556-591 (rope q, rope k,
 *                              append, attention; no rope without a table,
 *                              :556/:566)
 *       orc_decode_step_shared, orc_prefill_q
 *                           <- include/molot/forward.h:554-558, 578-591 and
 *                              :370-375, 394-398 (a layer reading another
 *                              layer's KV: q norm and rope, no append)
 *       orc_attn_prefill    <- include/molot/gemm.h:409-446 (causal prefill:
 *                              scalar expf, double denominator)
 *       orc_quantize_q8_row <- include/molot/quant.h:34-50 (quantize_q8_row), the
 *                              row quantizer of this build's Q8 KV cache
 *                              (kv_dtype ORC_KV_Q8, see below)
 *       orc_rmsnorm         <- include/molot/norm.h:9-28 (weights) and
 *                              :82-96 (w == NULL: rmsnorm_plain)
 *       orc_decode_step_norm <- include/molot/forward.h:554-591 with the
 *                              layer's norms: q and k per head
 *                              (rms_per_head, :138-140), v over all its
 *                              nkv*d values (:563), before RoPE
 *     Threading follows ThreadPool::parallel_for (thread_pool.h:54-89): a
 *     static contiguous split of the query heads, via OpenMP schedule(static).
 *
 *  2. A double-precision brute force (orc_attn_decode_f64), the formulation
 *     of the reference's own attention check (bench/bench.cc:195-213), used
 *     to pin (1) independently of its summation order.
 *
 * Pinning (see tests/test_oracle.py): the vexp known-answer points of
 * bench/bench.cc:220-234; the attention check of bench/bench.cc:186-218;
 * the compiled reference headers (oracle/_ref) where they build; golden
 * fixtures under tests/golden/; and closed-form invariants (rotation norm,
 * relative-position property, constant V, equal keys, window == slice,
 * permutation invariance, layout invariance).
 */
#include "attn_oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* bf16 helpers: include/molot/quant.h:186-198 (RNE, no NaN special case) */

static inline float orc_bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t orc_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

void orc_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16(in[i]);
}

/* ------------------------------------------------------------------ */
/* a2: inv_freq[i] = 1 / base^(2i/d) in fp32 (attn.h:31-33, model.h:546) */
void orc_rope_inv_freq(float base, int d, float* out) {
  for (int i = 0; i < d / 2; ++i) out[i] = 1.0f / powf(base, (2.0f * (float)i) / (float)d);
}

/* a1: NEOX half-split rotation, pair i = (x[i], x[i+d/2]).  The angle is the
 * fp32 product pos*inv_freq[i] (attn.h:22); sin/cos are full-range. */
void orc_rope_apply(float* x, int d, int pos, const float* inv_freq) {
  int h = d / 2;
  for (int i = 0; i < h; ++i) {
    float ang = (float)pos * inv_freq[i];
    float c = cosf(ang), s = sinf(ang);
    float x0 = x[i], x1 = x[i + h];
    x[i] = x0 * c - x1 * s;
    x[i + h] = x0 * s + x1 * c;
  }
}

/* Apply a1 to `nheads` consecutive heads of width d (forward.h:556-558). */
void orc_rope_apply_heads(float* x, int nheads, int d, int pos, const float* inv_freq) {
  for (int hh = 0; hh < nheads; ++hh) orc_rope_apply(x + (size_t)hh * d, d, pos, inv_freq);
}

/* ------------------------------------------------------------------ */
/* a5: vector exp, restated from its mathematics (norm.h:35-47):
 *   x <- clamp(x, -88, 88);  k = round_nearest_even(x * log2 e);
 *   r = x - k ln2 (one fused multiply-add);
 *   p = Taylor-5 of e^r in Horner form (1/120, 1/24, 1/6, 1/2, 1, 1);
 *   result = p * 2^k  (exact scaling). */
static inline float orc_vexp1(float x) {
  if (x < -88.0f) x = -88.0f;
  if (x > 88.0f) x = 88.0f;
  float k = nearbyintf(x * 1.4426950409f);
  float r = fmaf(-k, 0.6931471806f, x);
  float p = 1.0f / 120;
  p = fmaf(p, r, 1.0f / 24);
  p = fmaf(p, r, 1.0f / 6);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)k);
}

void orc_vexp16(const float* in, float* out) {
  for (int i = 0; i < 16; ++i) out[i] = orc_vexp1(in[i]);
}

void orc_vexp(const float* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_vexp1(in[i]);
}

/* 16-wide horizontal add, pairwise halves like a 512->256->128->... fold. */
static inline float orc_hsum16(const float* a) {
  float b[8], c[4];
  for (int i = 0; i < 8; ++i) b[i] = a[i] + a[i + 8];
  for (int i = 0; i < 4; ++i) c[i] = b[i] + b[i + 4];
  return (c[0] + c[2]) + (c[1] + c[3]);
}

/* a4: sum a_i b_i with 16 interleaved accumulators, horizontal fold, tail. */
float orc_dot(const float* a, const float* b, int n) {
  float acc[16] = {0};
  int i = 0;
  for (; i + 16 <= n; i += 16)
    for (int l = 0; l < 16; ++l) acc[l] = fmaf(a[i + l], b[i + l], acc[l]);
  float tail = 0;
  for (; i < n; ++i) tail += a[i] * b[i];
  return orc_hsum16(acc) + tail;
}

/* rmsnorm (norm.h:9-28): the sum of squares with the 16-lane FMA
 * accumulation of the reference's AVX512 loop (as orc_dot), mean = sum/n,
 * inv = 1/sqrt(mean + eps) in fp32, y = (x*inv)*w.  w == NULL is
 * rmsnorm_plain (norm.h:82-96): y = x*inv.  y may alias x. */
void orc_rmsnorm(const float* x, const float* w, float* y, int n, float eps) {
  const float inv = 1.0f / sqrtf(orc_dot(x, x, n) / (float)n + eps);
  for (int i = 0; i < n; ++i) y[i] = w ? (x[i] * inv) * w[i] : x[i] * inv;
}

/* ------------------------------------------------------------------ */
/* K/V addressing.  One description covers every layout on the path:
 *   contiguous:  row t of head h at base + t*tok_stride + h*head_stride
 *                (token-major cache [n][nkv*d]: tok=nkv*d, head=d;
 *                 head-major bench layout [nkv][n][d]: tok=d, head=n*d)
 *   paged:       block b = block_table[t / page]; row at
 *                base + b*block_stride + h*head_stride + (t % page)*tok_stride
 */
typedef struct {
  const void* k;
  const void* v;
  int kv_dtype;
  int64_t tok_stride, head_stride, block_stride;
  const int32_t* block_table; /* NULL => contiguous */
  int page;
  int nkv, d; /* Q8: scale addressing */
} orc_kv_t;

/* ------------------------------------------------------------------ */
/* Q8 KV cache (ORC_KV_Q8).  The reference planned an int8 KV cache
 * (its DESIGN.md:48, exp/README.md:36-39 "kv_q8, deferred") but never fixed
 * a format; this build's is its own Q8_0 row quantizer applied per KV head
 * row: orc_quantize_q8_row.  Byte layouts:
 *   token-major: row t = [nkv][d] int8, then nkv fp32 scales, padded to 16
 *                bytes: orc_q8_row_bytes(nkv, d) bytes per token;
 *   paged:       block = [nkv][page][d] int8, then [nkv][page] fp32 scales:
 *                orc_q8_block_bytes(nkv, d, page) bytes per block.
 * A row dequantizes as q_i * s. */
int orc_q8_row_bytes(int nkv, int d) { return nkv * d + ((4 * nkv + 15) & ~15); }
int64_t orc_q8_block_bytes(int nkv, int d, int page) {
  return (int64_t)nkv * page * d + (int64_t)4 * nkv * page;
}

/* quantize_q8_row (quant.h:34-50) on one row of d values: s = absmax/127
 * (1 when that is not > 0), q_i = clamp(nearbyint(x_i / s), -127, 127). */
void orc_quantize_q8_row(const float* x, int d, int8_t* q, float* s) {
  float amax = 0;
  for (int i = 0; i < d; ++i) amax = amax > fabsf(x[i]) ? amax : fabsf(x[i]);
  float sc = amax / 127.0f;
  if (!(sc > 0)) sc = 1.0f;
  *s = sc;
  for (int i = 0; i < d; ++i) {
    int v = (int)nearbyintf(x[i] / sc);
    q[i] = (int8_t)(v > 127 ? 127 : (v < -127 ? -127 : v));
  }
}

/* Token t of a token-major Q8 cache from its nkv rows x [nkv][d]. */
void orc_q8_store_token(void* base, int64_t t, const float* x, int nkv, int d) {
  uint8_t* row = (uint8_t*)base + t * orc_q8_row_bytes(nkv, d);
  for (int h = 0; h < nkv; ++h)
    orc_quantize_q8_row(x + (size_t)h * d, d, (int8_t*)row + (size_t)h * d,
                        (float*)(row + (size_t)nkv * d) + h);
}

/* Tokens 0..n-1 of a token-major Q8 cache from rows x [n][nkv*d]. */
void orc_q8_store_tokens(void* base, int64_t n, const float* x, int nkv, int d) {
  for (int64_t t = 0; t < n; ++t) orc_q8_store_token(base, t, x + t * (size_t)nkv * d, nkv, d);
}

/* The strides of a Q8 cache are its byte layout's (the callers' element
 * strides describe fp32/bf16 layouts); head-major Q8 is not a layout here. */
static orc_kv_t orc_kv_make(const void* K, const void* V, int kv_dtype, int64_t tok,
                            int64_t head, int64_t block, const int32_t* bt, int page, int nkv,
                            int d) {
  orc_kv_t kv = {K, V, kv_dtype, tok, head, block, bt, page, nkv, d};
  if (kv_dtype == ORC_KV_Q8) {
    if (bt) {
      kv.tok_stride = d;
      kv.head_stride = (int64_t)page * d;
      kv.block_stride = orc_q8_block_bytes(nkv, d, page);
    } else {
      kv.tok_stride = orc_q8_row_bytes(nkv, d);
      kv.head_stride = d;
    }
  }
  return kv;
}

static inline int64_t orc_row_off(const orc_kv_t* kv, int h, int t) {
  if (!kv->block_table) return (int64_t)t * kv->tok_stride + (int64_t)h * kv->head_stride;
  int64_t b = kv->block_table[t / kv->page];
  return b * kv->block_stride + (int64_t)h * kv->head_stride +
         (int64_t)(t % kv->page) * kv->tok_stride;
}

/* Fetch row (h, t) of K or V as fp32 into `dst` (d floats). */
static inline const float* orc_row(const orc_kv_t* kv, int which, int h, int t, int d,
                                   float* dst) {
  const void* base = which ? kv->v : kv->k;
  int64_t off = orc_row_off(kv, h, t);
  if (kv->kv_dtype == ORC_KV_F32) return (const float*)base + off;
  if (kv->kv_dtype == ORC_KV_Q8) {
    const int8_t* p = (const int8_t*)base + off;
    int64_t soff;
    if (kv->block_table) {
      const int64_t b = kv->block_table[t / kv->page];
      soff = b * kv->block_stride + (int64_t)kv->nkv * kv->page * kv->d +
             4 * ((int64_t)h * kv->page + t % kv->page);
    } else {
      soff = (int64_t)t * kv->tok_stride + (int64_t)kv->nkv * kv->d + 4 * (int64_t)h;
    }
    float sc;
    memcpy(&sc, (const uint8_t*)base + soff, 4);
    for (int j = 0; j < d; ++j) dst[j] = (float)p[j] * sc;
    return dst;
  }
  const uint16_t* p = (const uint16_t*)base + off;
  for (int j = 0; j < d; ++j) dst[j] = orc_bf16_to_f32(p[j]);
  return dst;
}

static inline int orc_t0(int pos_cur, int window) {
  return (window > 0 && pos_cur - window + 1 > 0) ? pos_cur - window + 1 : 0;
}

/* One query head, the 3-pass algorithm of attn.h:132-176:
 *   pass 1  s_t = dot(q, K_t) * scale, running max m (init -1e30)
 *   pass 2  e_t = vexp(s_t - m) for 16-wide chunks starting at t0, scalar
 *           expf tail; den accumulates one 16-wide fold per chunk
 *   pass 3  out = sum_t (e_t * (1/den)) * V_t  (weights normalised first) */
static void orc_head(const float* qh, const orc_kv_t* kv, int h, float* oh, int n, int d,
                     float scale, int t0, float* scores, float* rowbuf) {
  float m = -1e30f;
  for (int t = t0; t < n; ++t) {
    const float* kr = orc_row(kv, 0, h, t, d, rowbuf);
    float s = orc_dot(qh, kr, d) * scale;
    scores[t] = s;
    if (s > m) m = s;
  }
  float den = 0;
  int t = t0;
  for (; t + 16 <= n; t += 16) {
    float e[16];
    for (int l = 0; l < 16; ++l) e[l] = orc_vexp1(scores[t + l] - m);
    memcpy(scores + t, e, sizeof e);
    den += orc_hsum16(e);
  }
  for (; t < n; ++t) {
    scores[t] = expf(scores[t] - m);
    den += scores[t];
  }
  float inv = 1.0f / den;
  for (int j = 0; j < d; ++j) oh[j] = 0;
  for (int tt = t0; tt < n; ++tt) {
    float w = scores[tt] * inv;
    const float* vr = orc_row(kv, 1, h, tt, d, rowbuf);
    for (int j = 0; j < d; ++j) oh[j] = fmaf(vr[j], w, oh[j]);
  }
}

static int orc_threads(int nthreads) {
#ifdef _OPENMP
  return nthreads > 0 ? nthreads : omp_get_max_threads();
#else
  (void)nthreads;
  return 1;
#endif
}

/* a9 generalised: GQA over the described K/V, batch of one sequence.
 * kv head of query head h is h / (nq/nkv) (attn.h:131). */
void orc_attn_decode(const float* Q, const void* K, const void* V, float* O, int nq, int nkv,
                     int n, int d, float scale, int pos_cur, int window, int kv_dtype,
                     int64_t tok_stride, int64_t head_stride, int64_t block_stride,
                     const int32_t* block_table, int page, int nthreads) {
  const orc_kv_t kv = orc_kv_make(K, V, kv_dtype, tok_stride, head_stride, block_stride,
                                  block_table, page, nkv, d);
  int groups = nq / nkv;
  int t0 = orc_t0(pos_cur, window);
  int nt = orc_threads(nthreads);
  (void)nt;
#pragma omp parallel num_threads(nt)
  {
    float* scores = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    float* rowbuf = (float*)malloc(sizeof(float) * (size_t)d);
#pragma omp for schedule(static)
    for (int h = 0; h < nq; ++h)
      orc_head(Q + (size_t)h * d, &kv, h / groups, O + (size_t)h * d, n, d, scale, t0, scores,
               rowbuf);
    free(scores);
    free(rowbuf);
  }
}

/* Exact attn.h:125 signature over the token-major cache [n][nkv*qhd]. */
void orc_attn_decode_gqa_cache(const float* Q, const float* K, const float* V, float* O, int nq,
                               int nkv, int n, int qhd, float scale, int pos_cur, int window,
                               int nthreads) {
  orc_attn_decode(Q, K, V, O, nq, nkv, n, qhd, scale, pos_cur, window, ORC_KV_F32,
                  (int64_t)nkv * qhd, qhd, 0, NULL, 0, nthreads);
}

/* Batched paged decode (no reference counterpart: the reference has no
 * paged cache).  Sequence b has n_b = seq_lens[b] valid slots, current
 * position pos[b] (n_b - 1 when pos is NULL) and block row
 * block_table[b*max_blocks ...]; page layout [block][nkv][page][d]. */
void orc_attn_decode_paged(const float* Q, const void* Kp, const void* Vp, float* O,
                           const int32_t* block_table, const int32_t* seq_lens,
                           const int32_t* pos, int B, int max_blocks, int nq, int nkv, int d,
                           int page, float scale, int window, int kv_dtype, int nthreads) {
  for (int b = 0; b < B; ++b) {
    int n = seq_lens[b];
    int p = pos ? pos[b] : n - 1;
    orc_attn_decode(Q + (size_t)b * nq * d, Kp, Vp, O + (size_t)b * nq * d, nq, nkv, n, d,
                    scale, p, window, kv_dtype, d, (int64_t)page * d, (int64_t)nkv * page * d,
                    block_table + (size_t)b * max_blocks, page, nthreads);
  }
}

/* forward.h:556-591 for one layer: rope q heads and k heads at `pos`,
 * append k (rotated) and v into slot `slot` of the token-major cache
 * (bf16-rounded when kv_dtype is bf16), then attention over n = slot + 1.
 * inv_freq NULL: a layer without RoPE (an empty L.freq, model.h:535-536),
 * whose q and k forward.h:556 and :566 leave unrotated. */
void orc_decode_step(float* q, float* k_new, const float* v_new, void* Kc, void* Vc, float* O,
                     int nq, int nkv, int d, int slot, int pos, const float* inv_freq,
                     float scale, int window, int kv_dtype, int nthreads) {
  if (inv_freq) {
    orc_rope_apply_heads(q, nq, d, pos, inv_freq);
    orc_rope_apply_heads(k_new, nkv, d, pos, inv_freq);
  }
  size_t S = (size_t)nkv * d;
  if (kv_dtype == ORC_KV_F32) {
    memcpy((float*)Kc + (size_t)slot * S, k_new, S * 4);
    memcpy((float*)Vc + (size_t)slot * S, v_new, S * 4);
  } else if (kv_dtype == ORC_KV_Q8) {
    orc_q8_store_token(Kc, slot, k_new, nkv, d);
    orc_q8_store_token(Vc, slot, v_new, nkv, d);
  } else {
    orc_f32_to_bf16_array(k_new, (uint16_t*)Kc + (size_t)slot * S, (int64_t)S);
    orc_f32_to_bf16_array(v_new, (uint16_t*)Vc + (size_t)slot * S, (int64_t)S);
  }
  orc_attn_decode(q, Kc, Vc, O, nq, nkv, slot + 1, d, scale, pos, window, kv_dtype, (int64_t)S,
                  d, 0, NULL, 0, nthreads);
}

/* forward.h:554-591 with the layer's norms: q heads RMS-normed with q_norm
 * (forward.h:554), k heads with k_norm (:562), v by the RMS of all its
 * nkv*d values when v_norm (:563), then orc_decode_step.  NULL weights skip
 * that norm.  v_new is left unchanged (the normed copy is appended). */
void orc_decode_step_norm(float* q, float* k_new, const float* v_new, void* Kc, void* Vc,
                          float* O, int nq, int nkv, int d, int slot, int pos,
                          const float* q_norm, const float* k_norm, int v_norm, float eps,
                          const float* inv_freq, float scale, int window, int kv_dtype,
                          int nthreads) {
  const size_t S = (size_t)nkv * d;
  float* v = (float*)malloc(S * sizeof(float));
  memcpy(v, v_new, S * sizeof(float));
  if (q_norm)
    for (int h = 0; h < nq; ++h) orc_rmsnorm(q + (size_t)h * d, q_norm, q + (size_t)h * d, d, eps);
  if (k_norm)
    for (int h = 0; h < nkv; ++h)
      orc_rmsnorm(k_new + (size_t)h * d, k_norm, k_new + (size_t)h * d, d, eps);
  if (v_norm) orc_rmsnorm(v, NULL, v, (int)S, eps);
  orc_decode_step(q, k_new, v, Kc, Vc, O, nq, nkv, d, slot, pos, inv_freq, scale, window,
                  kv_dtype, nthreads);
  free(v);
}

/* The query prologue of one token of a layer without its own KV
 * (forward.h:554-558 / :370-375): q heads RMS-normed with q_norm (NULL:
 * none), then rotated at pos when inv_freq is given.  Rows [M][nq][d], row m
 * at pos0 + m. */
void orc_prefill_q(float* q, int nq, int d, int M, int pos0, const float* q_norm, float eps,
                   const float* inv_freq) {
  for (int m = 0; m < M; ++m) {
    float* qm = q + (size_t)m * nq * d;
    if (q_norm)
      for (int h = 0; h < nq; ++h)
        orc_rmsnorm(qm + (size_t)h * d, q_norm, qm + (size_t)h * d, d, eps);
    if (inv_freq) orc_rope_apply_heads(qm, nq, d, pos0 + m, inv_freq);
  }
}

/* forward.h:554-558 and :578-591 for a layer that reads another layer's KV
 * (L.has_kv false): the query prologue at pos, then attention over the n
 * slots of the source cache (token-major, any kv_dtype); nothing appended. */
void orc_decode_step_shared(float* q, const void* Kc, const void* Vc, float* O, int nq, int nkv,
                            int d, int n, int pos, const float* q_norm, float eps,
                            const float* inv_freq, float scale, int window, int kv_dtype,
                            int nthreads) {
  orc_prefill_q(q, nq, d, 1, pos, q_norm, eps, inv_freq);
  const int64_t tok = kv_dtype == ORC_KV_Q8 ? orc_q8_row_bytes(nkv, d) : (int64_t)nkv * d;
  orc_attn_decode(q, Kc, Vc, O, nq, nkv, n, d, scale, pos, window, kv_dtype, tok, d, 0, NULL, 0,
                  nthreads);
}

/* Causal prefill attention (gemm.h:409-446) over the token-major cache
 * [N][nkv*d] that already holds the M new tokens.  Query m of head h sits at
 * position pos0 + m and attends slots [t0, nn): t0 from the window at that
 * position (clamped to N), nn = min(pos0 + m + 1, N).  Per (h, m):
 * s_t = dot(q, K_t) * scale with a running max (init -1e30); e_t =
 * expf(s_t - max) -- the scalar libm exp, not the vector exp of the decode
 * path -- summed in double; inv = (float)(1/den); out = sum_t V_t*(e_t*inv)
 * in fp32 over t in order.  Parallel over (head, query) like the
 * reference's parallel_for over nq*M.  bf16 caches (no reference
 * counterpart) are widened. */
void orc_attn_prefill(const float* Qm, const void* K, const void* V, float* Om, int nq, int nkv,
                      int M, int N, int d, float scale, int pos0, int window, int kv_dtype,
                      int nthreads) {
  const orc_kv_t kv = orc_kv_make(K, V, kv_dtype, (int64_t)nkv * d, d, 0, NULL, 0, nkv, d);
  const int G = nq / nkv;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
#pragma omp parallel
  {
    float* scores = (float*)malloc((size_t)(N > 0 ? N : 1) * sizeof(float));
    float* rowbuf = (float*)malloc((size_t)d * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t hm = 0; hm < (int64_t)nq * M; ++hm) {
      const int h = (int)(hm / M), m = (int)(hm % M);
      const int kvh = h / G;
      const int pos = pos0 + m;
      int t0 = orc_t0(pos, window);
      if (t0 > N) t0 = N;
      const int nn = pos + 1 < N ? pos + 1 : N;
      const float* qh = Qm + ((size_t)m * nq + h) * d;
      float* oh = Om + ((size_t)m * nq + h) * d;
      float mx = -1e30f;
      for (int t = t0; t < nn; ++t) {
        const float s = orc_dot(qh, orc_row(&kv, 0, kvh, t, d, rowbuf), d) * scale;
        scores[t] = s;
        if (s > mx) mx = s;
      }
      double den = 0;
      for (int t = t0; t < nn; ++t) {
        scores[t] = expf(scores[t] - mx);
        den += scores[t];
      }
      const float inv = (float)(1.0 / den);
      for (int j = 0; j < d; ++j) oh[j] = 0;
      for (int t = t0; t < nn; ++t) {
        const float w = scores[t] * inv;
        const float* vr = orc_row(&kv, 1, kvh, t, d, rowbuf);
        for (int j = 0; j < d; ++j) oh[j] += vr[j] * w;
      }
    }
    free(scores);
    free(rowbuf);
  }
}

/* ------------------------------------------------------------------ */
/* Double-precision brute force (the formulation of bench/bench.cc:195-213,
 * carried out entirely in double).  Same K/V description as above. */
void orc_attn_decode_f64(const float* Q, const void* K, const void* V, double* O, int nq,
                         int nkv, int n, int d, double scale, int pos_cur, int window,
                         int kv_dtype, int64_t tok_stride, int64_t head_stride,
                         int64_t block_stride, const int32_t* block_table, int page,
                         int nthreads) {
  const orc_kv_t kv = orc_kv_make(K, V, kv_dtype, tok_stride, head_stride, block_stride,
                                  block_table, page, nkv, d);
  int groups = nq / nkv;
  int t0 = orc_t0(pos_cur, window);
  int nt = orc_threads(nthreads);
  (void)nt;
#pragma omp parallel num_threads(nt)
  {
    double* s = (double*)malloc(sizeof(double) * (size_t)(n > 0 ? n : 1));
    float* rowbuf = (float*)malloc(sizeof(float) * (size_t)d);
#pragma omp for schedule(static)
    for (int h = 0; h < nq; ++h) {
      int kvh = h / groups;
      const float* qh = Q + (size_t)h * d;
      double* oh = O + (size_t)h * d;
      double m = -INFINITY;
      for (int t = t0; t < n; ++t) {
        const float* kr = orc_row(&kv, 0, kvh, t, d, rowbuf);
        double dot = 0;
        for (int j = 0; j < d; ++j) dot += (double)qh[j] * (double)kr[j];
        s[t] = dot * scale;
        if (s[t] > m) m = s[t];
      }
      double den = 0;
      for (int t = t0; t < n; ++t) {
        s[t] = exp(s[t] - m);
        den += s[t];
      }
      for (int j = 0; j < d; ++j) oh[j] = 0;
      for (int t = t0; t < n; ++t) {
        const float* vr = orc_row(&kv, 1, kvh, t, d, rowbuf);
        double w = s[t] / den;
        for (int j = 0; j < d; ++j) oh[j] += w * (double)vr[j];
      }
    }
    free(s);
    free(rowbuf);
  }
}
