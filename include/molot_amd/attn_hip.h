/*
 * molot_amd: MI355X (gfx950) fused RoPE + GQA decode attention, C ABI.
 *
 * Drop-in boundary for the single-token decode-attention step of the Molot
 * runtime.  Every entry point takes plain pointers and sizes, is asynchronous
 * on the HIP stream it is given (`stream` is a hipStream_t; NULL = the null
 * stream), and returns 0 or a non-zero status (molot_hip_strerror() names
 * it): no exceptions cross this ABI.  Device buffers are allocated and owned
 * by the caller; the library never frees or retains them.  The library keeps
 * one internal workspace per device (split-K partials, grown on demand).
 *
 * Layouts (d = head dim, element type fp32 or bf16 per `kv_dtype`):
 *   q, o            [nq][d] fp32, query head h uses KV head h / (nq/nkv)
 *   KV cache        token-major [cap][nkv*d]: slot t of head h at
 *                   t*nkv*d + h*d  (include/molot/attn.h:122-124,
 *                   include/molot/forward.h:48-51)
 *   head-major      [nkv][n][d] (include/molot/attn.h:111-112)
 *   paged           [block][nkv][page][d], block_table[b][max_blocks]
 *                   (no reference counterpart: the reference cache is not
 *                   paged)
 * Head dims: every decode, shared-KV and prefill entry takes any even d
 * from 2 to 512 for fp32 and bf16 caches (attn.h and gemm.h take any qhd,
 * attn.h:99, :174, gemm.h:409-446; gemma4's global layers are 512 wide,
 * model.h:562-564) and any d from 4 to 512 that is a multiple of 4 for Q8
 * caches (4-byte aligned code rows); anything else returns MOLOT_ENOTSUP
 * before launching.
 * Semantics (include/molot/attn.h:125-177): n = valid slots after the
 * append, window <= 0 attends [0, n), otherwise [t0, n) with
 * t0 = max(0, pos_cur - window + 1); an empty range yields o = 0.
 *
 * RoPE tables: every entry that rotates takes inv_freq, a device table of
 * d/2 floats (the layer's L.freq, include/molot/model.h:530-549).  Except
 * for molot_hip_rope_apply, inv_freq may be NULL: the layer has no RoPE
 * (an empty L.freq, model.h:535-536), and q and k pass unrotated, as
 * forward.h:373, :381, :556 and :566 skip rope_apply for such layers.
 */
#ifndef MOLOT_AMD_ATTN_HIP_H_
#define MOLOT_AMD_ATTN_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* KV element types. */
#define MOLOT_KV_F32 0
#define MOLOT_KV_BF16 1 /* RNE-rounded as include/molot/quant.h:192-198 */
/* Q8: each KV head row of d values is quantized as quantize_q8_row
 * (include/molot/quant.h:34-50): fp32 scale s = absmax/127 (1 when not > 0),
 * int8 codes clamp(nearbyint(x/s), -127, 127); it dequantizes as code * s.
 * The reference plans an int8 KV cache (its DESIGN.md:48, exp/README.md:36-39)
 * without fixing a layout; this library's layouts, in bytes:
 *   token-major  row t = [nkv][d] codes, then nkv fp32 scales, padded to 16
 *                bytes: molot_hip_q8_row_bytes(nkv, d) bytes per token;
 *   paged        block = [nkv][page][d] codes, then [nkv][page] fp32 scales:
 *                molot_hip_q8_block_bytes(nkv, d, page) bytes per block.
 * Q8 runs on head dims that are multiples of 4 up to 512 (MOLOT_ENOTSUP
 * otherwise; 64 and 128 feed the matrix cores, the others the vector-ALU
 * kernel); the head-major entry points take no Q8 cache (MOLOT_EINVAL). */
#define MOLOT_KV_Q8 2

/* Bytes of one token of a token-major Q8 cache, and of one paged Q8 block. */
int molot_hip_q8_row_bytes(int nkv, int d);
int64_t molot_hip_q8_block_bytes(int nkv, int d, int page);

/* Status codes besides hipError_t values (which are positive). */
#define MOLOT_OK 0
#define MOLOT_EINVAL (-22)  /* bad shape / argument */
#define MOLOT_ENOTSUP (-95) /* shape the kernels are not built for */
#define MOLOT_ENOSPC (-28)  /* append beyond the cache capacity */
#define MOLOT_ENOWS (-16)   /* workspace not sized for a launch being captured in a graph */
#define MOLOT_E2BIG (-7)    /* partials exceed the no-allocation entry point's scratch */

const char* molot_hip_strerror(int status);
/* Library version string ("molot_amd <major>.<minor>"). */
const char* molot_hip_version(void);

/* Host-side table: out[i] = 1 / base^(2i/d), i < d/2, computed in fp32 with
 * powf.  Replaces rope_inv_freq, include/molot/attn.h:31-33 (same formula as
 * the per-layer table of include/molot/model.h:546). */
void molot_rope_inv_freq(float base, int d, float* out);

/* In-place RoPE of `nheads` consecutive heads of x[nheads][d] at position
 * `pos` (NEOX half-split pairs (i, i+d/2), fp32 angle pos*inv_freq[i]).
 * Replaces rope_apply, include/molot/attn.h:19-28, as called per head at
 * include/molot/forward.h:556-558 and :566-568.  inv_freq: device [d/2]. */
int molot_hip_rope_apply(float* x, int nheads, int d, int pos, const float* inv_freq,
                         void* stream);

/* RoPE prologue + KV append of one decode step:
 *   rotate q[nq][d] in place; rotate k_new[nkv][d] (input, not modified) and
 *   store it, with v_new[nkv][d], into slot `slot` of the token-major cache
 *   K/V (fp32, or bf16 RNE when kv_dtype == MOLOT_KV_BF16).
 * Replaces include/molot/forward.h:556-558 (rope q), :566-568 (rope k) and
 * :571-575 (memcpy append).  The capacity check of forward.h:570 ("KV cache
 * full") is the caller's, as in the reference (see the C++ DeviceKV).
 * Stream-ordered before any attention launched afterwards on `stream`. */
int molot_hip_rope_append(float* q, const float* k_new, const float* v_new, void* K, void* V,
                          int nq, int nkv, int d, int slot, int pos, const float* inv_freq,
                          int kv_dtype, void* stream);

/* GQA decode attention over the token-major cache [n][nkv*qhd].
 * Replaces attn_decode_gqa_cache, include/molot/attn.h:125-127 (call site
 * include/molot/forward.h:589-590); the ThreadPool argument has no
 * counterpart.  K/V element type per kv_dtype (the reference is fp32). */
int molot_hip_attn_decode_gqa_cache(const float* Q, const void* K, const void* V, float* O,
                                    int nq, int nkv, int n, int qhd, float scale, int pos_cur,
                                    int window, int kv_dtype, void* stream);

/* GQA decode attention over the head-major layout [nkv][n][d], full prefix.
 * Replaces attn_decode_gqa, include/molot/attn.h:111-120 (the layout of the
 * reference benchmark, bench/bench.cc:357-383). */
int molot_hip_attn_decode_gqa(const float* Q, const void* K, const void* V, float* O, int nq,
                              int nkv, int n, int d, float scale, int kv_dtype, void* stream);

/* Head-major layout with a sliding window.
 * Replaces attn_decode_gqa_win, include/molot/attn.h:178-187. */
int molot_hip_attn_decode_gqa_win(const float* Q, const void* K, const void* V, float* O, int nq,
                                  int nkv, int n, int d, float scale, int pos_cur, int window,
                                  int kv_dtype, void* stream);

/* One head, contiguous K/V [n][d], with window.
 * Replaces attn_decode_head_win, include/molot/attn.h:57-101 (and
 * attn_decode_head, :104-107, with pos_cur = n, window = 0). */
int molot_hip_attn_decode_head_win(const float* Q, const void* K, const void* V, float* out,
                                   int n, int d, float scale, int pos_cur, int window,
                                   int kv_dtype, void* stream);

/* General strided form behind all of the above: row t of KV head h at
 * element offset t*tok_stride + h*head_stride.  At d = 64, 128, 256 and 512
 * the strides keep every row 16-byte aligned (16-byte loads); at other
 * head dims they are even (two-element loads); K, V, Q and O 16-byte
 * aligned (MOLOT_EINVAL otherwise).  Q8: the token-major Q8 layout only,
 * tok_stride = molot_hip_q8_row_bytes(nkv, d) and head_stride = d (bytes). */
int molot_hip_attn_decode_strided(const float* Q, const void* K, const void* V, float* O, int nq,
                                  int nkv, int n, int d, int64_t tok_stride, int64_t head_stride,
                                  float scale, int pos_cur, int window, int kv_dtype,
                                  void* stream);

/* One full decode layer-step: molot_hip_rope_append into slot `slot`, then
 * attention over n = slot + 1 at pos_cur = pos.  q is rotated in place and
 * O receives the attention output.  Replaces the block
 * include/molot/forward.h:556-591 for a layer that owns its KV. */
int molot_hip_decode_step(float* q, const float* k_new, const float* v_new, void* K, void* V,
                          float* O, int nq, int nkv, int d, int slot, int pos,
                          const float* inv_freq, float scale, int window, int kv_dtype,
                          void* stream);

/* molot_hip_decode_step that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, semantics and kernels as
 * molot_hip_decode_step; the split-K partials go to a fixed 4 MiB device
 * array that each device holds from module load to process end, always
 * merged by the combine kernel.  A shape whose partials exceed it returns
 * MOLOT_E2BIG (for example 32q/8kv/d128 uses 0.5 MiB at any context under
 * the automatic chunking; 64q/8kv/d128 bf16 1 MiB).  Every call on a
 * device shares that array: calls that overlap on one device (two streams,
 * or two host threads) race and must be ordered by the caller. */
int molot_hip_decode_step_noalloc(float* q, const float* k_new, const float* v_new, void* K,
                                  void* V, float* O, int nq, int nkv, int d, int slot, int pos,
                                  const float* inv_freq, float scale, int window, int kv_dtype,
                                  void* stream);

/* molot_hip_decode_step with the layer's norms fused in, in forward.h's
 * order (include/molot/forward.h:554-568): each q head and each new k head
 * RMS-normed with the weights q_norm[d] / k_norm[d]
 * (Runner::rms_per_head, forward.h:138-140 -> rmsnorm, norm.h:9-28:
 * y = (x * 1/sqrt(mean(x^2) + eps)) * w), v RMS-normed over all its nkv*d
 * values without weights when v_norm != 0 (rmsnorm_plain, norm.h:82-96,
 * forward.h:563), then RoPE, append and attention.  A NULL weight pointer
 * skips that norm; eps >= 0 (the model's hp.eps). */
int molot_hip_decode_step_norm(float* q, const float* k_new, const float* v_new, void* K,
                               void* V, float* O, int nq, int nkv, int d, int slot, int pos,
                               const float* q_norm, const float* k_norm, int v_norm, float eps,
                               const float* inv_freq, float scale, int window, int kv_dtype,
                               void* stream);

/* Batched decode over a paged cache (continuous batching; no reference
 * counterpart).  Q/O [B][nq][d] fp32; K/V pages [num_blocks][nkv][page][d];
 * sequence b attends slots [t0_b, seq_lens[b]) through
 * block_table[b*max_blocks + t/page], with pos_cur = pos[b] (seq_lens[b]-1
 * when pos is NULL).  All index arrays are device int32. */
int molot_hip_attn_decode_paged(const float* Q, const void* K, const void* V, float* O,
                                const int32_t* block_table, const int32_t* seq_lens,
                                const int32_t* pos, int B, int max_blocks, int max_seq_len,
                                int nq, int nkv, int d, int page, float scale, int window,
                                int kv_dtype, void* stream);

/* One fused decode step per sequence over the paged cache: RoPE of q (in
 * place) and of k_new, append of k/v at slot seq_lens[b]-1 of sequence b,
 * attention over [t0_b, seq_lens[b]).  seq_lens counts the new token.  The
 * batched counterpart of molot_hip_decode_step (include/molot/forward.h:556-591
 * per sequence; the paged cache has no reference counterpart). */
int molot_hip_decode_step_paged(float* q, const float* k_new, const float* v_new, void* K,
                                void* V, float* O, const int32_t* block_table,
                                const int32_t* seq_lens, const int32_t* pos, int B,
                                int max_blocks, int max_seq_len, int nq, int nkv, int d, int page,
                                const float* inv_freq, float scale, int window, int kv_dtype,
                                void* stream);

/* molot_hip_decode_step_paged with the layer's norms, per sequence, as
 * molot_hip_decode_step_norm (include/molot/forward.h:554-568). */
int molot_hip_decode_step_paged_norm(float* q, const float* k_new, const float* v_new, void* K,
                                     void* V, float* O, const int32_t* block_table,
                                     const int32_t* seq_lens, const int32_t* pos, int B,
                                     int max_blocks, int max_seq_len, int nq, int nkv, int d,
                                     int page, const float* q_norm, const float* k_norm,
                                     int v_norm, float eps, const float* inv_freq, float scale,
                                     int window, int kv_dtype, void* stream);

/* RoPE + append for the paged cache: q[B][nq][d] rotated in place at pos[b];
 * k_new/v_new [B][nkv][d] (k rotated) written to slot seq_lens[b]-1 of
 * sequence b through its block table. */
int molot_hip_rope_append_paged(float* q, const float* k_new, const float* v_new, void* K,
                                void* V, const int32_t* block_table, const int32_t* seq_lens,
                                const int32_t* pos, int B, int max_blocks, int nq, int nkv, int d,
                                int page, const float* inv_freq, int kv_dtype, void* stream);

/* Causal prefill attention, counterpart of attn_prefill_gqa
 * (include/molot/gemm.h:409-446, called at forward.h:394-399): Qm and Om
 * [M][nq][d] fp32; K/V the token-major cache [N][nkv*d] holding the M new
 * tokens; query m sits at position pos0 + m and attends slots
 * [t0, min(pos0 + m + 1, N)), t0 = max(0, pos - window + 1) for window > 0.
 * A query with no slot gets O = 0.  scale as given. */
int molot_hip_attn_prefill_gqa(const float* Qm, const void* K, const void* V, float* Om, int nq,
                               int nkv, int M, int N, int d, float scale, int pos0, int window,
                               int kv_dtype, void* stream);

/* One layer's prefill of M prompt tokens, forward.h:367-399: per token the
 * layer's norms (as molot_hip_decode_step_norm; NULL weights / v_norm = 0
 * skip them) and RoPE of q (in place, [M][nq][d]) and k_new ([M][nkv][d]),
 * append of k/v at slots slot0 .. slot0+M-1 (positions pos0 ..), then
 * causal prefill attention over N = slot0 + M into O [M][nq][d]. */
int molot_hip_prefill_step(float* q, const float* k_new, const float* v_new, void* K, void* V,
                           float* O, int nq, int nkv, int d, int M, int slot0, int pos0,
                           const float* q_norm, const float* k_norm, int v_norm, float eps,
                           const float* inv_freq, float scale, int window, int kv_dtype,
                           void* stream);

/* molot_hip_prefill_step for one sequence of a paged cache (no reference
 * counterpart): its M prompt rows go to slots slot0 .. slot0+M-1 through its
 * block-table row block_row[max_blocks] (device int32) into pages
 * [num_blocks][nkv][page][d]; the attention reads the same pages. */
int molot_hip_prefill_step_paged(float* q, const float* k_new, const float* v_new, void* K,
                                 void* V, float* O, const int32_t* block_row, int max_blocks,
                                 int page, int nq, int nkv, int d, int M, int slot0, int pos0,
                                 const float* q_norm, const float* k_norm, int v_norm, float eps,
                                 const float* inv_freq, float scale, int window, int kv_dtype,
                                 void* stream);

/* Layers that read another layer's KV cache (L.has_kv false: the shared-KV
 * tail of include/molot/model.h:562-583).  The reference norms and rotates
 * q as for any layer and attends the source layer's cache kv[L.kv_src]
 * over its n = src.n slots, appending nothing (forward.h:554-558, 578-591
 * for decode; :370-375, 394-398 for prefill). */

/* Decode step of such a layer over a token-major cache: q[nq][d] RMS-normed
 * per head with q_norm (NULL: no norm; eps >= 0) and rotated at pos
 * (inv_freq NULL: no RoPE), in place, then attention over the source cache
 * K/V's n slots (n >= 1: forward.h:580 throws "shared KV empty" at 0) into
 * O, with pos_cur = pos.  One launch (two with a split context that cannot
 * be merged in the launch). */
int molot_hip_decode_step_shared(float* q, const void* K, const void* V, float* O, int nq,
                                 int nkv, int d, int n, int pos, const float* q_norm, float eps,
                                 const float* inv_freq, float scale, int window, int kv_dtype,
                                 void* stream);

/* The same per sequence of a batch over a paged cache (no reference
 * counterpart): sequence b attends the rows [t0_b, seq_lens[b]) of the
 * source layer's pages (seq_lens[b] >= 1), pos[b] as in
 * molot_hip_attn_decode_paged. */
int molot_hip_decode_step_paged_shared(float* q, const void* K, const void* V, float* O,
                                       const int32_t* block_table, const int32_t* seq_lens,
                                       const int32_t* pos, int B, int max_blocks, int max_seq_len,
                                       int nq, int nkv, int d, int page, const float* q_norm,
                                       float eps, const float* inv_freq, float scale, int window,
                                       int kv_dtype, void* stream);

/* Query prologue of a prefill without an append (forward.h:370-375 for a
 * layer without its own KV): the nq heads of row m of q[M][nq][d] RMS-normed
 * with q_norm and rotated at pos0 + m, in place; NULL skips either.  Then
 * molot_hip_attn_prefill_gqa (or _paged) over the source layer's cache is
 * forward.h:394-398. */
int molot_hip_prefill_q(float* q, int nq, int d, int M, int pos0, const float* q_norm, float eps,
                        const float* inv_freq, void* stream);

/* molot_hip_attn_prefill_gqa over one sequence of a paged cache (no
 * reference counterpart): pages [num_blocks][nkv][page][d] through its
 * block-table row block_row[max_blocks] (device int32), N <= max_blocks*page
 * valid slots. */
int molot_hip_attn_prefill_paged(const float* Qm, const void* K, const void* V, float* Om,
                                 const int32_t* block_row, int max_blocks, int page, int nq,
                                 int nkv, int M, int N, int d, float scale, int pos0, int window,
                                 int kv_dtype, void* stream);

/* The exponential of the split-K merges (the chunk weights e^(m_c - M),
 * the device expf), applied elementwise (x, y device [n]).  Counterpart of
 * exp_avx512_ps, include/molot/norm.h:35-47, exposed so its accuracy can be
 * checked against the reference's known-answer points
 * (bench/bench.cc:220-234). */
int molot_hip_vexp(const float* x, float* y, int64_t n, void* stream);

/* The exponential the decode and prefill kernels take of every attention
 * probability: y = 2^(x * log2(e)), the product rounded once to fp32 and
 * one hardware v_exp_f32 (the kernels hold scores in base-2 units).  The
 * other counterpart of exp_avx512_ps (norm.h:35-47), exposed for the same
 * known-answer points; its relative error grows with |x| by the rounding
 * of x * log2(e), ~|x| * 2^-24. */
int molot_hip_prob_exp(const float* x, float* y, int64_t n, void* stream);

/* Process-wide settings (no reference counterpart; for measurement and
 * tests).  Each is an atomic that launches read when they are planned, so
 * setting one while other host threads launch is safe; it applies to
 * launches planned afterwards. */

/* Split-K chunk size in tokens (0 = automatic). */
void molot_hip_set_split_chunk(int tokens);

/* Workgroups per CU the split-K plan targets (0 = the plan's own). */
void molot_hip_set_tuning(int wgs_per_cu);

/* How a split context's chunk partials are merged.  in_launch = 0: by a
 * second kernel (combine_kernel) on the same stream.  in_launch = 1: inside
 * the attention launch, by the workgroup that completes a (sequence, KV
 * head group) slot, where the device dispatches workgroup i to XCD i % 8
 * (checked once per device) and the launch can keep a slot's chunks on one
 * XCD; other launches use the combine kernel.  in_launch < 0 (default):
 * in the launch for the fp32 vector-ALU kernel when the slots are a
 * multiple of 8 on a contiguous cache (every XCD busy) and the attended
 * context spans at least 8192 rows, else the combine kernel.  Both give the same result to
 * fp32 rounding.  If a launch ever found a slot's chunks on different XCDs
 * its merged output would be NaN rather than a stale merge. */
void molot_hip_set_merge(int in_launch);

/* How the prefill entries feed fp32 and Q8 caches to the matrix cores: K
 * and V as two fp16 pieces of each row scaled by a power of two (the scores
 * and PV), exact to fp32 rounding.
 * on = 1 (default): the attended keys of every KV head are split into
 * pieces once per launch, into a per-stream workspace of
 * 12 * nkv * (N - t0) * d bytes (at most 1 GiB; it grows outside stream
 * capture only, and the buffers it outgrows stay allocated, under 1 GiB in
 * all), and the attention kernel copies them into LDS.  on = 0, or when that
 * workspace is unavailable: the attention kernel splits each staged tile
 * itself.  Both give the same bits.  A Q8 cache at d = 256 always takes the
 * pieces (its matrix-core kernel has no per-tile split); without them it
 * runs on the vector-ALU kernel, each query row a sequence of its own (the
 * path of d = 512, of head dims that are not multiples of 8 and of Q8 caches
 * at head dims other than 64, 128 and 256), which agrees to fp32 rounding. */
void molot_hip_set_prefill_presplit(int on);

/* Order in which the waves of a workgroup take their chunk's row blocks.
 * dynamic = 1 (default): a wave takes the next free block when it has one
 * to spare, so faster-served waves take more; the fp32 summation order then
 * varies from run to run (results agree to rounding).  dynamic = 0: a fixed
 * order, bit-identical from run to run.  Process-wide. */
void molot_hip_set_block_order(int dynamic);

/* Kernel for bf16 KV caches with head dim 64 or 128.  mfma = 1 (default):
 * the matrix-core kernel (scores and PV on v_mfma_f32_16x16x32_bf16, q and
 * the probabilities split into three bf16 pieces each, fp32 accumulation);
 * mfma = 0: the vector-ALU kernel of the fp32 caches.  Both compute the
 * same softmax(q.K^T*scale).V to fp32 rounding.  Process-wide; for
 * comparisons and tests. */
void molot_hip_set_bf16_path(int mfma);

/* Launch profiling, the counterpart of the reference's MOLOT_PROFILE
 * attention timer (include/molot/forward.h:114-137, :588-591).
 * molot_hip_profile_begin(max_launches) starts recording: each attention
 * entry launched afterwards (outside graph capture, up to max_launches) has
 * its kernels launched with start/stop HIP events stamped by the dispatch
 * itself (hipExtLaunchKernelGGL).  molot_hip_profile_end() stops,
 * waits for the recorded events and returns the summed durations (ms) of
 * the attention kernel (*attn_ms over *launches launches) and of the
 * split-K combine kernel (*combine_ms over *combines launches that needed
 * one).  Process-wide; meant for measurement, not for concurrent callers. */
int molot_hip_profile_begin(int max_launches);
int molot_hip_profile_end(float* attn_ms, float* combine_ms, int* launches, int* combines);

/* Geometry of the calling thread's last attention launch: context chunks
 * per (sequence, KV head) (grid x; 1 = no combine kernel) and rows per
 * chunk.  Returns MOLOT_EINVAL before the thread's first launch. */
int molot_hip_last_plan(int* nchunks, int* chunk);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* MOLOT_AMD_ATTN_HIP_H_ */
