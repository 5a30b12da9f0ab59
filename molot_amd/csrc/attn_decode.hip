// MI355X (gfx950) fused RoPE + GQA decode attention.
//
// Kernels:
//   rope_append_kernel   RoPE of q (in place) and of the new k, append of the
//                        rotated k and v into the cache slot
//                        (include/molot/forward.h:556-575).
//   split_kernel         flash-decoding split-K attention: one workgroup per
//                        (KV head, GQA head subgroup, context chunk, sequence).
//                        Each K/V row is fetched from HBM once with 16-byte
//                        coalesced loads and consumed by every query head of
//                        the group held in registers; chunk scores live in
//                        LDS; the chunk's (max, sum, unnormalised o) partial
//                        is written for the combine
//                        (include/molot/attn.h:125-177 computes the same
//                        softmax(qK^T*scale)V in three passes per head).
//   combine_kernel       log-sum-exp merge of the chunk partials.
//
// All shapes are validated on the host before any launch.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <mutex>
#include <type_traits>
#include <utility>
#include <vector>

#include "molot_amd/attn_hip.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// KV element traits: one 16-byte vector = VW elements.
template <typename T>
struct KVT;

template <>
struct KVT<float> {
  static constexpr int VW = 4;
  using vec = f32x4;
  __device__ static __forceinline__ void unpack(const vec& v, float* x) {
    x[0] = v[0];
    x[1] = v[1];
    x[2] = v[2];
    x[3] = v[3];
  }
};

struct bf16_t {
  uint16_t bits;
};

template <>
struct KVT<bf16_t> {
  static constexpr int VW = 8;
  using vec = u32x4;
  __device__ static __forceinline__ void unpack(const vec& v, float* x) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(v[i] << 16);
      x[2 * i + 1] = __uint_as_float(v[i] & 0xFFFF0000u);
    }
  }
};

// Q8 codes (the row scale is applied by the kernel that reads them).
struct q8_t {
  int8_t code;
};

template <>
struct KVT<q8_t> {
  static constexpr int VW = 16;
  using vec = u32x4;
  __device__ static __forceinline__ void unpack(const vec& v, float* x) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[4 * i] = (float)(int8_t)(v[i] & 0xFF);
      x[4 * i + 1] = (float)(int8_t)((v[i] >> 8) & 0xFF);
      x[4 * i + 2] = (float)(int8_t)((v[i] >> 16) & 0xFF);
      x[4 * i + 3] = (float)((int32_t)v[i] >> 24);
    }
  }
};

// K/V rows are read exactly once per step: non-temporal 16-byte loads (the
// streaming hint measurably raises the sustained HBM read rate on gfx950).
// Q8 rows excepted: the KV heads of a token share 128-byte lines (head rows
// of d bytes at t*R + h*d, the token's scales after them), so a line one
// head's workgroup fetched has to stay in the L2 for its neighbour's.
template <typename T>
__device__ __forceinline__ typename KVT<T>::vec load16(const T* p) {
  if constexpr (std::is_same<T, q8_t>::value)
    return *reinterpret_cast<const typename KVT<T>::vec*>(p);
  else
    return __builtin_nontemporal_load(reinterpret_cast<const typename KVT<T>::vec*>(p));
}

// A 16-byte vector of row elements [e, e + VW) of a head row of dh
// elements (dh even, possibly not a multiple of VW), read as VW/2 pieces of
// two elements (Q8: VW/4 pieces of four codes, dh a multiple of 4).  Pieces
// at or past dh read the row's first piece instead: they stay inside the
// row, their K products meet q's zero padding and their V products land in
// output elements that are never stored.
template <typename T>
__device__ __forceinline__ typename KVT<T>::vec load_pad(const T* row, int e, int dh) {
  using V = typename KVT<T>::vec;
  constexpr int PB = 2 * (int)sizeof(T);  // bytes per two-element piece
  V v;
  const char* r = reinterpret_cast<const char*>(row);
  if constexpr (std::is_same<T, q8_t>::value) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ee = e + 4 * i < dh ? e + 4 * i : 0;
      v[i] = *reinterpret_cast<const uint32_t*>(r + ee);  // plain: heads share lines
    }
  } else if constexpr (PB == 8) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int ee = e + 2 * i < dh ? e + 2 * i : 0;
      const f32x2 x = __builtin_nontemporal_load(reinterpret_cast<const f32x2*>(r + ee * 4));
      v[2 * i] = x[0];
      v[2 * i + 1] = x[1];
    }
  } else {
    static_assert(PB == 4, "fp32 or bf16 rows");
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ee = e + 2 * i < dh ? e + 2 * i : 0;
      v[i] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(r + ee * 2));
    }
  }
  return v;
}

// Round-to-nearest-even fp32 -> bf16 (include/molot/quant.h:192-198).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// ---------------------------------------------------------------------------
// Q8 rows (the Q8_0 row quantizer of include/molot/quant.h:34-50, applied
// per KV head row): s = absmax/127 (1 when that is not > 0), codes
// clamp(nearbyint(x/s), -127, 127); a row dequantizes as code * s.  The
// divisions are IEEE-correct (hipcc's default for fp32 / ), so the codes and
// scales are the reference quantizer's bit for bit on the same fp32 input.
__device__ __forceinline__ float q8_scale(float amax) {
  const float s = amax / 127.0f;
  return s > 0.f ? s : 1.0f;
}
__device__ __forceinline__ int q8_code(float x, float s) {
  const int v = (int)__builtin_rintf(x / s);
  return v > 127 ? 127 : (v < -127 ? -127 : v);
}

// ---------------------------------------------------------------------------
// Cross-lane sums.  Lanes are grouped in aligned groups of N; every lane of
// a group receives the group's sum.  Groups up to 16 use DPP within a row
// (quad_perm xor1, quad_perm xor2, row_half_mirror, row_mirror: after the
// quad steps every lane holds its quad's sum, and each mirror pairs a lane
// with one in the other half of its 8/16-lane block).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// x of lanes l and l ^ 16 (xor16), or l and l ^ 32 (xor32), as the pair
// (lower lane's, upper lane's) in every lane: v_permlane16_swap and
// v_permlane32_swap exchange 16- or 32-lane rows of two registers, so with
// both operands x they leave the lower row's x in the first and the upper
// row's in the second, in both rows (checked lane by lane on the GPU).
// Reducing the pair gives every lane the same operands in the same order,
// where a shuffle would take two LDS round trips.
__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// x combined with lane l ^ OFF's x (a sum in the shuffle's operand order)
template <int OFF>
__device__ __forceinline__ float sum_xor(float x) {
  if constexpr (OFF == 16) return sum_xor16(x);
  else if constexpr (OFF == 32) return sum_xor32(x);
  else return x + __shfl_xor(x, OFF);
}
template <int OFF>
__device__ __forceinline__ float max_xor(float x) {
  if constexpr (OFF == 16) return max_xor16(x);
  else if constexpr (OFF == 32) return max_xor32(x);
  else return fmaxf(x, __shfl_xor(x, OFF));
}

template <int N>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (N >= 2) v = fmaxf(v, dpp_f<0xB1>(v));
  if constexpr (N >= 4) v = fmaxf(v, dpp_f<0x4E>(v));
  if constexpr (N >= 8) v = fmaxf(v, dpp_f<0x141>(v));
  if constexpr (N >= 16) v = fmaxf(v, dpp_f<0x140>(v));
  if constexpr (N >= 32) v = max_xor16(v);
  if constexpr (N >= 64) v = max_xor32(v);
  return v;
}

template <int N>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (N >= 2) v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  if constexpr (N >= 4) v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  if constexpr (N >= 8) v += dpp_f<0x141>(v);  // row_half_mirror
  if constexpr (N >= 16) v += dpp_f<0x140>(v); // row_mirror
  if constexpr (N >= 32) v = sum_xor16(v);
  if constexpr (N >= 64) v = sum_xor32(v);
  return v;
}

// Wave-wide max / sum with DPP only (no LDS round trips): the quad and
// mirror steps reduce each row of 16 lanes, row_bcast:15 and row_bcast:31
// carry the partial results up to lane 63, which readlane broadcasts.
template <bool MAX>
__device__ __forceinline__ float wave_reduce(float v) {
  auto op = [](float x, float y) { return MAX ? fmaxf(x, y) : x + y; };
  v = op(v, dpp_f<0xB1>(v));   // quad_perm [1,0,3,2]
  v = op(v, dpp_f<0x4E>(v));   // quad_perm [2,3,0,1]
  v = op(v, dpp_f<0x141>(v));  // row_half_mirror
  v = op(v, dpp_f<0x140>(v));  // row_mirror
  // row_bcast:15 into rows 1 and 3, row_bcast:31 into rows 2 and 3; rows
  // outside the mask keep their value (old = v)
  v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(MAX ? -INFINITY : 0.f),
                                                       __float_as_int(v), 0x142, 0xA, 0xF,
                                                       false)));
  v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(MAX ? -INFINITY : 0.f),
                                                       __float_as_int(v), 0x143, 0xC, 0xF,
                                                       false)));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// exp used by the split-K merges (full-accuracy device expf).
__device__ __forceinline__ float softmax_exp(float x) { return expf(x); }

// The decode kernels' softmax runs in base 2: a score is q.k * scale*log2(e)
// (the matrix-core kernel pre-scales q, the vector-ALU kernel each score), so
// p = 2^(s - m) is one v_exp_f32 (relative error ~|s - m| * 2^-24, within
// the reference's own exp, exp_avx512_ps at 1.5e-6).  The maxima leave the
// kernels in natural units (m * ln 2) for the split-K merges.
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }
// A running max moves only when a score exceeds it by more than kLazyMax
// (p <= 2^8 otherwise): o and l always share the max they were formed with,
// so the result is exact either way, and most blocks skip the rescale.
constexpr float kLazyMax = 8.f;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16_pair_exact(float a, float b) {
  const bf16x2_t p = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, p);
}

// split3 of two values at once: each piece of the pair is one
// v_cvt_pk_bf16_f32 (round to nearest even, as split3), element a in the
// low half.  The same pieces as split3 on each value.
__device__ __forceinline__ uint32_t bf16_pair(float a, float b) { return bf16_pair_exact(a, b); }
__device__ __forceinline__ void split3x2(float a, float b, uint32_t& hi, uint32_t& mid,
                                         uint32_t& lo) {
  // The residuals are taken of a and b as rounded to fp32: a product that
  // formed them (a Q8 code times its scale, q times the score scale) must
  // not fuse into the first subtraction, or the pieces would split the
  // unrounded product and differ between the kernels that form a and b
  // differently.
#pragma clang fp contract(off)
  hi = bf16_pair(a, b);
  float ra = a - __uint_as_float(hi << 16), rb = b - __uint_as_float(hi & 0xFFFF0000u);
  mid = bf16_pair(ra, rb);
  ra -= __uint_as_float(mid << 16);
  rb -= __uint_as_float(mid & 0xFFFF0000u);
  lo = bf16_pair(ra, rb);
}

// Two fp16 pieces of a row scaled by a power of two: with the row's largest
// |x| in [2^(ex-1), 2^ex) (frexpf of it), y = x * 2^(14-ex) has |y| < 2^14,
// hi = fp16(y), lo = fp16(y - hi), each rounded to nearest even.  hi + lo
// holds y to 2^-22 of |y| while |y| >= 2^-3 (lo a normal fp16), and to
// 2^-25 absolute below (2^-38 of the row's largest |y|); the scaling is
// exact.  y's unit is 2^(ex-14) (f16_row_unit), the factor that takes a
// dot product of such pieces back.  Non-finite values make NaN pieces.
__device__ __forceinline__ int f16_row_shift(float amax) {
  int ex = 0;
  (void)frexpf(amax, &ex);
  return 14 - ex;
}
__device__ __forceinline__ float f16_row_unit(int shift) { return ldexpf(1.f, -shift); }
__device__ __forceinline__ uint32_t f16_pair(float a, float b) {
  const _Float16 ha = (_Float16)a, hb = (_Float16)b;
  return (uint32_t)__builtin_bit_cast(uint16_t, ha) |
         ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
}
__device__ __forceinline__ void split2h(float a, float b, int shift, uint32_t& hi, uint32_t& lo) {
#pragma clang fp contract(off)
  const float ya = ldexpf(a, shift), yb = ldexpf(b, shift);
  hi = f16_pair(ya, yb);
  const float ra = ya - (float)__builtin_bit_cast(_Float16, (uint16_t)(hi & 0xFFFFu));
  const float rb = yb - (float)__builtin_bit_cast(_Float16, (uint16_t)(hi >> 16));
  lo = f16_pair(ra, rb);
}
// V rows (the prefill's PV operand): the same split, with the unit kept a
// normal float (shift <= 120: 2^-120 and up; rows below 2^-106 keep fewer
// bits, as fp32 denormals would) and 0 for a row of zeros, which then
// weighs nothing and never sets a tile's largest unit.
__device__ __forceinline__ int f16_vrow_shift(float amax) { return min(f16_row_shift(amax), 120); }
__device__ __forceinline__ float f16_vrow_unit(float amax, int shift) {
  return amax > 0.f ? f16_row_unit(shift) : 0.f;
}

// ---------------------------------------------------------------------------
// RoPE + append.
struct RopeArgs {
  float* q;            // [B][nq][d], rotated in place (may be null)
  const float* k_new;  // [B][nkv][d]
  const float* v_new;  // [B][nkv][d]
  void* K;
  void* V;
  const float* inv_freq;  // [d/2]
  const int32_t* block_table;
  const int32_t* seq_lens;
  const int32_t* pos_arr;
  const float* q_norm;  // [d] q RMS-norm weights (NULL: no q norm)
  const float* k_norm;  // [d] k RMS-norm weights (NULL: no k norm)
  int64_t tok_stride, head_stride, block_stride;
  int nq, nkv, d, slot, pos, max_blocks, page, kv_dtype, append;
  int v_norm;           // RMS-norm v over all nkv*d values, no weights
  float eps;
  int tokens;           // grid row b = token b of a prefill: slot + b at pos + b
  int64_t sc_off, sc_head;  // Q8 scales, as AttnArgs::sc_off / sc_head
  // prefill over an fp32 or Q8 cache: the appended rows also leave their
  // pieces (as pf_split_kernel writes them) at row slot - pc_T0 of
  // [K, V][nkv][3][pc_R][d], when that row lies in [0, pc_R) (NULL: none)
  uint16_t* pieces;
  int pc_T0, pc_R;
};

// Sum over the workgroup (at most 16 waves); every thread gets the total.
__device__ __forceinline__ float block_sum(float v, float* sh) {
  v = group_sum<64>(v);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = 0.f;
  for (int k = 0; k < (int)((blockDim.x + 63) >> 6); ++k) t += sh[k];
  __syncthreads();
  return t;
}

// Maximum over the workgroup (at most 16 waves); every thread gets it.
__device__ __forceinline__ float block_max(float v, float* sh) {
  v = group_max<64>(v);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = sh[0];
  for (int k = 1; k < (int)((blockDim.x + 63) >> 6); ++k) t = fmaxf(t, sh[k]);
  __syncthreads();
  return t;
}

// One workgroup per (head of q or k, sequence); one thread per rotation pair.
// Angle is the fp32 product pos*inv_freq[i] (include/molot/attn.h:22); its
// sine and cosine are evaluated in double and rounded, i.e. a full-range,
// correctly rounded (barring double rounding) fp32 sin/cos.  With the
// layer's norms (forward.h:554, 562-563) a head is RMS-normed before its
// rotation: (x * 1/sqrt(mean(x^2) + eps)) * w (include/molot/norm.h:9-28),
// and v by the RMS of all nkv*d values of the sequence's v (norm.h:82-96).
__global__ void rope_append_kernel(RopeArgs a) {
  __shared__ float sh[16];
  const int hh = blockIdx.x;
  const int b = blockIdx.y;
  const int half = a.d >> 1;
  const int i = threadIdx.x;
  const bool act = i < half;  // the reductions need every thread
  const int ic = act ? i : 0;
  int pos = a.pos;
  int slot = a.slot;
  if (a.seq_lens) {
    slot = a.seq_lens[b] - 1;
    pos = a.pos_arr ? a.pos_arr[b] : slot;
  } else if (a.tokens) {
    slot += b;
    pos += b;
  }
  const bool rot = a.inv_freq != nullptr;  // a NoPE layer (inv_freq NULL) is not rotated
  float c = 1.f, s = 0.f;
  if (rot) {
    const float ang = (float)pos * a.inv_freq[ic];
    double sd, cd;
    sincos((double)ang, &sd, &cd);
    c = (float)cd;
    s = (float)sd;
  }
  auto rms_inv = [&](float ss, int n) { return 1.0f / sqrtf(ss / (float)n + a.eps); };
  if (hh < a.nq) {
    if (!a.q) return;
    float* x = a.q + ((int64_t)b * a.nq + hh) * a.d;
    float x0 = act ? x[i] : 0.f, x1 = act ? x[i + half] : 0.f;
    if (a.q_norm) {
      const float inv = rms_inv(block_sum(x0 * x0 + x1 * x1, sh), a.d);
      x0 = x0 * inv * a.q_norm[ic];
      x1 = x1 * inv * a.q_norm[ic + half];
    }
    if (act) {
      x[i] = rot ? x0 * c - x1 * s : x0;
      x[i + half] = rot ? x0 * s + x1 * c : x1;
    }
    return;
  }
  if (!a.append) return;
  const int kh = hh - a.nq;
  const float* kx = a.k_new + ((int64_t)b * a.nkv + kh) * a.d;
  const float* vx = a.v_new + ((int64_t)b * a.nkv + kh) * a.d;
  float k0 = act ? kx[i] : 0.f, k1 = act ? kx[i + half] : 0.f;
  float v0 = act ? vx[i] : 0.f, v1 = act ? vx[i + half] : 0.f;
  if (a.k_norm) {
    const float inv = rms_inv(block_sum(k0 * k0 + k1 * k1, sh), a.d);
    k0 = k0 * inv * a.k_norm[ic];
    k1 = k1 * inv * a.k_norm[ic + half];
  }
  if (a.v_norm) {
    const float* vall = a.v_new + (int64_t)b * a.nkv * a.d;
    float part = 0.f;
    for (int j = i; j < a.nkv * a.d; j += blockDim.x) part = fmaf(vall[j], vall[j], part);
    const float inv = rms_inv(block_sum(part, sh), a.nkv * a.d);
    v0 *= inv;
    v1 *= inv;
  }
  const float r0 = rot ? k0 * c - k1 * s : k0;  // 0 on the threads past the pairs
  const float r1 = rot ? k0 * s + k1 * c : k1;
  float ks = 0.f, vs = 0.f;
  if (a.kv_dtype == MOLOT_KV_Q8) {  // uniform: every thread takes the maxima
    ks = q8_scale(block_max(fmaxf(fabsf(r0), fabsf(r1)), sh));
    vs = q8_scale(block_max(fmaxf(fabsf(v0), fabsf(v1)), sh));
  }
  if (!act) return;
  // element (Q8: byte) offset of the row, and (Q8) of its scale
  int64_t off, soff;
  if (a.block_table) {
    const int64_t blk = a.block_table[(int64_t)b * a.max_blocks + slot / a.page];
    off = blk * a.block_stride + (int64_t)kh * a.head_stride + (int64_t)(slot % a.page) * a.tok_stride;
    soff = blk * a.block_stride + a.sc_off + kh * a.sc_head + 4 * (int64_t)(slot % a.page);
  } else {
    off = (int64_t)slot * a.tok_stride + (int64_t)kh * a.head_stride;
    soff = (int64_t)slot * a.tok_stride + a.sc_off + kh * a.sc_head;
  }
  if (a.kv_dtype == MOLOT_KV_Q8) {
    int8_t* kd = (int8_t*)a.K + off;
    int8_t* vd = (int8_t*)a.V + off;
    kd[i] = (int8_t)q8_code(r0, ks);
    kd[i + half] = (int8_t)q8_code(r1, ks);
    vd[i] = (int8_t)q8_code(v0, vs);
    vd[i + half] = (int8_t)q8_code(v1, vs);
    if (i == 0) {
      *(float*)((char*)a.K + soff) = ks;
      *(float*)((char*)a.V + soff) = vs;
    }
  } else if (a.kv_dtype == MOLOT_KV_F32) {
    float* kd = (float*)a.K + off;
    float* vd = (float*)a.V + off;
    kd[i] = r0;
    kd[i + half] = r1;
    vd[i] = v0;
    vd[i + half] = v1;
  } else {
    uint16_t* kd = (uint16_t*)a.K + off;
    uint16_t* vd = (uint16_t*)a.V + off;
    kd[i] = f32_to_bf16(r0);
    kd[i + half] = f32_to_bf16(r1);
    vd[i] = f32_to_bf16(v0);
    vd[i + half] = f32_to_bf16(v1);
  }
}

// The prefill's RoPE/append (and the q prologue): one workgroup of 4 waves
// per token instead of one per (head, token).  The token's sine and cosine
// are taken once (in double, as rope_append_kernel) into LDS; wave w takes
// heads w, w + 4, ..., lane l the pairs l, l + 64, ... of a head, so a head's
// norm sum and Q8 maximum stay in its wave.  Sums run as rope_append_kernel's
// (per 64 pairs, added in order), so rows of d <= 128 come out bit-identical.
// 2048 tokens of 32q/8kv/d128: 81920 single-wave workgroups became 2048.
constexpr int kRopeTokThreads = 256;
constexpr int kRopeMaxPairs = 1024;  // d <= 2048
template <int KMAX>  // pair groups of 64 a head holds at most (d <= 128 KMAX)
__global__ __launch_bounds__(kRopeTokThreads) void rope_append_tok_kernel(RopeArgs a) {
  __shared__ float cs_s[kRopeMaxPairs], sn_s[kRopeMaxPairs];
  __shared__ float sh[16];
  const int b = blockIdx.x;
  const int half = a.d >> 1;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int pos = a.pos + b, slot = a.slot + b;
  const bool rot = a.inv_freq != nullptr;
  for (int i = tid; rot && i < half; i += kRopeTokThreads) {
    const float ang = (float)pos * a.inv_freq[i];
    double sd, cd;
    sincos((double)ang, &sd, &cd);
    cs_s[i] = (float)cd;
    sn_s[i] = (float)sd;
  }
  auto rms_inv = [&](float ss, int n) { return 1.0f / sqrtf(ss / (float)n + a.eps); };
  // the v norm: one RMS over the token's nkv*d values (wave 0, stride 64)
  if (a.append && a.v_norm && w == 0) {
    const float* vall = a.v_new + (int64_t)b * a.nkv * a.d;
    float part = 0.f;
    for (int j = lane; j < a.nkv * a.d; j += 64) part = fmaf(vall[j], vall[j], part);
    part = group_sum<64>(part);
    if (lane == 0) sh[0] = rms_inv(part, a.nkv * a.d);
  }
  __syncthreads();
  const float vinv = a.append && a.v_norm ? sh[0] : 1.f;
  const int nk = (half + 63) / 64;  // pair groups of 64 per head
  // Each wave walks its heads with the next head's rows loaded before the
  // current head's stores go out (heads own disjoint rows), so a wave waits
  // for one load latency in all rather than one per head.
  auto load_q = [&](int hh, float* y0, float* y1) {
    const float* x = a.q + ((int64_t)b * a.nq + hh) * a.d;
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      if (k >= nk) break;
      const int j = lane + 64 * k;
      y0[k] = j < half ? x[j] : 0.f;
      y1[k] = j < half ? x[j + half] : 0.f;
    }
  };
  if (a.q) {
    float x0[KMAX], x1[KMAX], n0[KMAX] = {}, n1[KMAX] = {};
    if (w < a.nq) load_q(w, n0, n1);
    for (int hh = w; hh < a.nq; hh += kRopeTokThreads / 64) {
#pragma unroll
      for (int k = 0; k < KMAX; ++k) {
        x0[k] = n0[k];
        x1[k] = n1[k];
      }
      if (hh + kRopeTokThreads / 64 < a.nq) load_q(hh + kRopeTokThreads / 64, n0, n1);
      float* x = a.q + ((int64_t)b * a.nq + hh) * a.d;
      float ss = 0.f;
      if (a.q_norm) {
#pragma unroll
        for (int k = 0; k < KMAX; ++k) {
          if (k >= nk) break;
          ss += group_sum<64>(x0[k] * x0[k] + x1[k] * x1[k]);
        }
      }
      const float inv = a.q_norm ? rms_inv(ss, a.d) : 1.f;
#pragma unroll
      for (int k = 0; k < KMAX; ++k) {
        if (k >= nk) break;
        const int j = lane + 64 * k;
        if (j >= half) continue;
        float y0 = x0[k], y1 = x1[k];
        if (a.q_norm) {
          y0 = y0 * inv * a.q_norm[j];
          y1 = y1 * inv * a.q_norm[j + half];
        }
        x[j] = rot ? y0 * cs_s[j] - y1 * sn_s[j] : y0;
        x[j + half] = rot ? y0 * sn_s[j] + y1 * cs_s[j] : y1;
      }
    }
  }
  if (!a.append) return;
  // KV heads: wave w takes heads kh with (nq + kh) % 4 == w
  auto load_kv = [&](int kh, float* k0, float* k1, float* v0, float* v1) {
    const float* kx = a.k_new + ((int64_t)b * a.nkv + kh) * a.d;
    const float* vx = a.v_new + ((int64_t)b * a.nkv + kh) * a.d;
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      if (k >= nk) break;
      const int j = lane + 64 * k;
      k0[k] = j < half ? kx[j] : 0.f;
      k1[k] = j < half ? kx[j + half] : 0.f;
      v0[k] = j < half ? vx[j] : 0.f;
      v1[k] = j < half ? vx[j + half] : 0.f;
    }
  };
  constexpr int kWaves = kRopeTokThreads / 64;
  const int kh0 = ((w - a.nq) % kWaves + kWaves) % kWaves;
  float nk0[KMAX] = {}, nk1[KMAX] = {}, nv0[KMAX] = {}, nv1[KMAX] = {};
  if (kh0 < a.nkv) load_kv(kh0, nk0, nk1, nv0, nv1);
  for (int kh = kh0; kh < a.nkv; kh += kWaves) {
    float r0[KMAX], r1[KMAX], v0[KMAX], v1[KMAX];
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      r0[k] = nk0[k];
      r1[k] = nk1[k];
      v0[k] = nv0[k] * vinv;
      v1[k] = nv1[k] * vinv;
    }
    if (kh + kWaves < a.nkv) load_kv(kh + kWaves, nk0, nk1, nv0, nv1);
    float ss = 0.f;
    if (a.k_norm) {
#pragma unroll
      for (int k = 0; k < KMAX; ++k) {
        if (k >= nk) break;
        ss += group_sum<64>(r0[k] * r0[k] + r1[k] * r1[k]);
      }
    }
    const float kinv = a.k_norm ? rms_inv(ss, a.d) : 1.f;
    float kmax = 0.f, vmax = 0.f;
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      if (k >= nk) break;
      const int j = lane + 64 * k;
      const int jc = j < half ? j : 0;
      float k0 = r0[k], k1 = r1[k];
      if (a.k_norm) {
        k0 = k0 * kinv * a.k_norm[jc];
        k1 = k1 * kinv * a.k_norm[jc + half];
      }
      r0[k] = rot ? k0 * cs_s[jc] - k1 * sn_s[jc] : k0;  // 0 past the pairs
      r1[k] = rot ? k0 * sn_s[jc] + k1 * cs_s[jc] : k1;
      kmax = fmaxf(kmax, fmaxf(fabsf(r0[k]), fabsf(r1[k])));
      vmax = fmaxf(vmax, fmaxf(fabsf(v0[k]), fabsf(v1[k])));
    }
    float ks = 0.f, vs = 0.f;
    if (a.kv_dtype == MOLOT_KV_Q8) {
      ks = q8_scale(group_max<64>(kmax));
      vs = q8_scale(group_max<64>(vmax));
    }
    int64_t off, soff;
    if (a.block_table) {
      const int64_t blk = a.block_table[slot / a.page];
      off = blk * a.block_stride + (int64_t)kh * a.head_stride + (int64_t)(slot % a.page) * a.tok_stride;
      soff = blk * a.block_stride + a.sc_off + kh * a.sc_head + 4 * (int64_t)(slot % a.page);
    } else {
      off = (int64_t)slot * a.tok_stride + (int64_t)kh * a.head_stride;
      soff = (int64_t)slot * a.tok_stride + a.sc_off + kh * a.sc_head;
    }
    #pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      if (k >= nk) break;
      const int j = lane + 64 * k;
      if (j >= half) continue;
      if (a.kv_dtype == MOLOT_KV_Q8) {
        int8_t* kd = (int8_t*)a.K + off;
        int8_t* vd = (int8_t*)a.V + off;
        kd[j] = (int8_t)q8_code(r0[k], ks);
        kd[j + half] = (int8_t)q8_code(r1[k], ks);
        vd[j] = (int8_t)q8_code(v0[k], vs);
        vd[j + half] = (int8_t)q8_code(v1[k], vs);
      } else if (a.kv_dtype == MOLOT_KV_F32) {
        float* kd = (float*)a.K + off;
        float* vd = (float*)a.V + off;
        kd[j] = r0[k];
        kd[j + half] = r1[k];
        vd[j] = v0[k];
        vd[j + half] = v1[k];
      } else {
        uint16_t* kd = (uint16_t*)a.K + off;
        uint16_t* vd = (uint16_t*)a.V + off;
        kd[j] = f32_to_bf16(r0[k]);
        kd[j + half] = f32_to_bf16(r1[k]);
        vd[j] = f32_to_bf16(v0[k]);
        vd[j + half] = f32_to_bf16(v1[k]);
      }
    }
    if (a.kv_dtype == MOLOT_KV_Q8 && lane == 0) {
      *(float*)((char*)a.K + soff) = ks;
      *(float*)((char*)a.V + soff) = vs;
    }
    // the row's pieces for the prefill (of the cached values: fp32 as
    // stored, Q8 as code * scale), the bits pf_split_kernel writes: K and
    // V as two fp16 pieces of the row scaled by a power of two (split2h,
    // the row's unit at float pr of the head's third piece)
    const int pr = slot - a.pc_T0;
    if (a.pieces && a.kv_dtype != MOLOT_KV_BF16 && pr >= 0 && pr < a.pc_R) {
      const int64_t pstride = (int64_t)a.pc_R * a.d;  // one piece of one head
      auto cached = [&](float x, float sc) {
        return a.kv_dtype == MOLOT_KV_Q8 ? (float)q8_code(x, sc) * sc : x;
      };
      float kpm = 0.f, vpm = 0.f;  // the rows' largest |k| and |v| as cached
#pragma unroll
      for (int k = 0; k < KMAX; ++k) {
        if (k >= nk) break;
        if (lane + 64 * k < half) {
          kpm = fmaxf(kpm, fmaxf(fabsf(cached(r0[k], ks)), fabsf(cached(r1[k], ks))));
          vpm = fmaxf(vpm, fmaxf(fabsf(cached(v0[k], vs)), fabsf(cached(v1[k], vs))));
        }
      }
      const int kshift = f16_row_shift(group_max<64>(kpm));
      vpm = group_max<64>(vpm);
      const int vshift = f16_vrow_shift(vpm);
      uint16_t* ok = a.pieces + (int64_t)kh * 3 * pstride + (int64_t)pr * a.d;
      uint16_t* ov = ok + (int64_t)a.nkv * 3 * pstride;
      if (lane == 0) {  // the units of a head's rows side by side in its third piece
        reinterpret_cast<float*>(ok - (int64_t)pr * a.d + 2 * pstride)[pr] = f16_row_unit(kshift);
        reinterpret_cast<float*>(ov - (int64_t)pr * a.d + 2 * pstride)[pr] =
            f16_vrow_unit(vpm, vshift);
      }
#pragma unroll
      for (int k = 0; k < KMAX; ++k) {
        if (k >= nk) break;
        const int j = lane + 64 * k;
        if (j >= half) continue;
        uint32_t pk[2], pv[2];
        split2h(cached(r0[k], ks), cached(r1[k], ks), kshift, pk[0], pk[1]);
        split2h(cached(v0[k], vs), cached(v1[k], vs), vshift, pv[0], pv[1]);
#pragma unroll
        for (int pc = 0; pc < 2; ++pc) {
          ok[pc * pstride + j] = (uint16_t)(pk[pc] & 0xFFFF);
          ok[pc * pstride + j + half] = (uint16_t)(pk[pc] >> 16);
          ov[pc * pstride + j] = (uint16_t)(pv[pc] & 0xFFFF);
          ov[pc * pstride + j + half] = (uint16_t)(pv[pc] >> 16);
        }
      }
    }
  }
}

// rope_append_tok_kernel for M tokens of head dim d (<= 2048).
int launch_rope_tok(const RopeArgs& r, int M, void* stream) {
  const int half = r.d / 2;
  auto k = half <= 64 ? rope_append_tok_kernel<1>
           : half <= 128 ? rope_append_tok_kernel<2>
                         : rope_append_tok_kernel<kRopeMaxPairs / 64>;
  hipLaunchKernelGGL(k, dim3(M), dim3(kRopeTokThreads), 0, (hipStream_t)stream, r);
  return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// Fused decode attention.
//
// Grid (nkv * subgroups, sequences, chunks).  Workgroup (h/sub, b, c) owns
// chunk c of the context rows of KV head h and the GH query heads
// hq0 .. hq0+GH-1 of that head's group: a paged cache's rows [tb, tb + cnt),
// a contiguous cache's 32-row groups c, c + nchunks, c + 2*nchunks, ... of the
// range.  The workgroups sharing (b, h/sub) form a "slot".
//   1. prologue: the first block(s) of K/V rows of every wave, then q of the
//      GH heads into LDS; with ROPE, q is rotated there, and the workgroup
//      holding the chunk that contains the new token rotates k_new and
//      rounds k/v to the cache type in LDS.  Every wave issues the same
//      loads on every path and the barriers order LDS only, so nothing waits
//      for the K/V blocks in flight before it has to;
//   2. every wave streams blocks of RB rows (NBUF blocks in flight); blocks
//      past the first NBUF per wave are claimed from a workgroup counter in
//      LDS, so waves that are served faster take more.  Scores of the GH
//      heads per K row (LPR lanes per row, DPP sums); online softmax per
//      wave (running max, rescale of the accumulators); probabilities through
//      a per-wave LDS slice to the PV lanes (LPR2 lanes per V row, 16 bytes
//      each);
//   3. the new token (ROPE, last chunk): folded in by wave 0 from LDS, and
//      stored into the cache slot n-1 by subgroup 0 as the kernel's last
//      step (no workgroup reads that slot in this launch);
//   4. the waves' (max, sum, o) are merged through LDS; every thread derives
//      its own outputs' chunk partial.  A single-chunk problem writes
//      o / sum (and the rotated q) directly;
//   5. otherwise the chunk partial (o, max, sum) goes to the workspace, and
//      combine_kernel, launched next on the same stream, merges the chunks
//      of every slot with log-sum-exp weights and writes O (and, with ROPE,
//      the rotated q, which chunk 0 leaves in the workspace: q is rotated in
//      place, so it is written back only after every workgroup has read it).
struct AttnArgs {
  const float* q;        // [B][nq][D]; un-rotated when the kernel applies RoPE
  float* q_out;          // [B][nq][D] rotated q (ROPE); written after every read of q
  const float* k_new;    // [B][nkv][D] fp32 (ROPE)
  const float* v_new;    // [B][nkv][D] fp32 (ROPE)
  void* k;               // KV cache
  void* v;
  const float* inv_freq; // [D/2] (ROPE)
  float* o;              // [B][nq][D]
  float* part_o;         // [slots][nchunks][GH*D] chunk partial o (split-K)
  float* part_ml;        // [slots][nchunks][GH][2] chunk partial (max, sum)
  float* qrot;           // [slots][GH*D] rotated q for the combine kernel (ROPE)
  void* ext_ws;          // host side only: caller-provided workspace (NULL: the library's)
  int64_t ext_ws_bytes;
  const int32_t* block_table;
  const int32_t* seq_lens;
  const int32_t* pos_arr;
  int64_t tok_stride, head_stride, block_stride;
  int nq, nkv, n, t0, pos, chunk, nchunks, max_blocks, page_shift, window;
  int dh;                // head dim as stored (< D: the kernel runs padded to its D)
  int dynamic;           // 1: waves claim blocks from a workgroup counter; 0: fixed order
  int chunk_fast;        // 1-D grid, the KV heads of a chunk on one XCD (Q8; see launch_pair)
  // Prefill rows (attention-only launches): "sequence" b is query row b of a
  // prompt, at position pos + b, attending [t0_b, min(pos + b + 1, n)) of the
  // one cache (contiguous, or the prompt's block-table row: max_blocks = 0),
  // t0_b from the window (include/molot/gemm.h:409-446).
  int pf;
  int nseq;              // chunk_fast: sequences of the launch
  // In-launch merge (see arrive_and_merge): every chunk of a slot runs on one
  // XCD, and the workgroup that completes a slot merges its chunk partials.
  int fold;              // ROPE: 1 = the step appends the new token (folded into the last
                         // chunk, slot n-1); 0 = q prologue only (a layer reading another
                         // layer's KV: all n slots come from the cache)
  unsigned long long* ctr;  // [slots] arrival words (arrive_and_merge), zero between launches
                            // (NULL: combine kernel)
  int xmap;              // 1-D grid of 8 * nchunks: slot id % 8 on XCD id % 8 (fewer than 8 slots)
  int slots;             // slots of the launch (xmap)
  int mrg;               // floats of LDS for the merge's chunk statistics (0: no in-launch merge)
  float scale;
  // the layer's norms of the fresh vectors (ROPE only; NULL / 0: none)
  const float* q_norm;   // [D] weights of the per-head q RMS norm
  const float* k_norm;   // [D] weights of the per-head k RMS norm
  int v_norm;            // RMS-norm v over all nkv*D values, no weights
  float eps;
  // Q8 caches: byte offset of head 0's fp32 row scales from the token's row
  // (token-major) or the block (paged), and the byte stride between heads'
  // scales; a paged block's scales step 4 bytes per slot
  int64_t sc_off, sc_head;
};

// Work mapping of one kernel instance.
//   LPR   lanes cooperating on one K row in the score loop (DPP sums across them)
//   RB    rows per wave block
//   NW    waves per workgroup
//   NBUF  blocks in flight per wave: 1 (load, then score) or 2 (one block is
//         scored while the next one's loads are outstanding)
template <int D, int GH, typename T, int LPR_, int RB_, int NW_, int NBUF_ = 1>
struct Cfg {
  static constexpr int NBUF = NBUF_;
  static_assert(NBUF == 1 || NBUF == 2, "one or two blocks in flight");
  static constexpr int VW = KVT<T>::VW;
  static constexpr int LPR = LPR_;
  static constexpr int NV = D / (LPR * VW);  // 16-byte vectors per lane per K row
  static constexpr int EPL = NV * VW;        // q elements per lane
  static constexpr int RPS = 64 / LPR;       // K rows per wave step
  // PV: a V row is LPR2 <= 64 lanes of NV2 16-byte vectors each (NV2 = 2
  // for fp32 rows of 512 elements); lane cs holds row elements
  // (v2*LPR2 + cs)*VW .. +VW-1, so each v2 reads LPR2*16 contiguous bytes
  static constexpr int NV2 = (D / VW + 63) / 64;
  static constexpr int LPR2 = D / (VW * NV2);  // lanes per V row
  static constexpr int AW = VW * NV2;          // o accumulators per head and lane
  static constexpr int RPI = 64 / LPR2;        // V rows per wave step
  static constexpr int RB = RB_;
  static constexpr int KS = RB / RPS;  // K steps per block
  static constexpr int VS = RB / RPI;  // V steps per block
  static constexpr int NW = NW_;
  static constexpr int NT = NW * 64;
  static constexpr int P = GH * D;
  // chunk partial: PP output pairs per thread (P > NT), Q threads per copy
  static constexpr int PP = (P + NT - 1) / NT;
  static constexpr int Q = P < NT ? P : NT;
  static_assert(NV >= 1 && D % (LPR * VW) == 0 && LPR <= 64, "bad score mapping");
  static_assert(LPR2 * VW * NV2 == D && LPR2 <= 64 && 64 % LPR2 == 0, "bad PV mapping");
  static_assert(RB % RPS == 0 && RB % RPI == 0, "bad block");
  static_assert(P % 64 == 0 || P <= NT, "pairs per phase");
};

// Default mapping: q registers (GH x D/LPR) kept at <= 32 where the 16-byte
// vector allows it; one block in flight per wave; 8-row blocks at two waves
// per SIMD where D <= 128 and the register estimate allows, else the block size with the
// most waves per SIMD; one workgroup per CU (NW = 4 x waves per SIMD, at
// most 16).
template <int D, int GH, typename T>
struct Tune {
  static constexpr int VW = KVT<T>::VW;
  static constexpr int lpr() {
    int l = D / VW < 8 ? D / VW : 8;  // Q8 at D = 64: 4 lanes of 16 codes a row
    while (GH * D / l > 32 && l < D / VW && l < 64) l *= 2;
    return l;
  }
  static constexpr int LPR = lpr();
  static constexpr int NV = D / (LPR * VW);
  static constexpr int NV2 = (D / VW + 63) / 64;
  static constexpr int RPS = 64 / LPR, RPI = 64 / (D / (VW * NV2));
  static constexpr int loads(int rb) { return (rb / RPS) * NV + (rb / RPI) * NV2; }
  static constexpr int regs(int rb) {  // one block of data + its addresses
    return GH * NV * VW + GH * VW * NV2 + 6 * loads(rb) + (rb / RPS) * GH + 3 * GH + 40;
  }
  static constexpr int wps(int rb) {
    const int r = (regs(rb) + 7) / 8 * 8;
    const int w = 512 / r;
    return w > 4 ? 4 : w;
  }
  static constexpr bool ok(int rb) {
    return rb % RPS == 0 && rb % RPI == 0 && loads(rb) <= 16 && wps(rb) >= 2;
  }
  // 8-row blocks and two waves per SIMD where the registers allow (D <= 128):
  // the same bytes in flight per CU as 4-row blocks at four waves per SIMD,
  // with half the waves to merge at the chunk's end (measured, 32q/8kv/d128
  // fp32: step 28.8 -> 27.3 us at n = 16385, 14.0 -> 13.3 us at n = 4097;
  // at d = 256, 8q/4kv with a 1024 window, 12 waves of 4-row blocks stay
  // faster: 9.3 against 9.6 us).
  // d = 512: the largest block whose loads fit at two waves per SIMD (fp32
  // 4 rows = 16 KB of K and V a wave, bf16 8 rows), else at one.
  static constexpr bool fits(int rb, int w) {
    return rb % RPS == 0 && rb % RPI == 0 && loads(rb) <= 16 && wps(rb) >= w;
  }
  static constexpr int rb() {
    if (D <= 128 && ok(8)) return 8;
    if (D > 256) {
      for (int w : {2, 1})
        for (int r : {16, 8, 4, 2, 1})
          if (fits(r, w)) return r;
    }
    int best = 0;
    for (int r : {16, 4})
      if (ok(r) && (best == 0 || wps(r) > wps(best))) best = r;
    if (best) return best;
    return RPS > RPI ? RPS : RPI;
  }
  static constexpr int RB = rb();
  static constexpr int nw() {
    const int w = RB == 8 ? 2 : (wps(RB) >= 1 ? wps(RB) : 1);
    int nw = 4 * w;
    // wave-merge buffer <= 32 KiB (64 KiB at d = 512, one workgroup a CU:
    // two waves per SIMD instead of one: 8q/2kv/d512 Q8 step
    // 32.7 -> 29.8 us, fp32 61.5 -> 60.9 us)
    while (nw > 4 && nw * GH * D > (D > 256 ? 16384 : 8192)) nw -= 4;
    return nw;
  }
  static constexpr int NW = nw();
  // d = 512 (fp32 and bf16) and d = 128 fp32: two blocks of half the rows
  // in flight, so a wave's next loads go out before it scores the current
  // block (same box, interleaved: 8q/2kv/d512 step fp32 60.9 -> 60.2 us,
  // bf16 36.4 -> 34.4 us; 32q/8kv/d128 fp32 at n = 4097 12.11 -> 11.99 us,
  // at n = 16385 25.88 against 25.85 us; two 8-row blocks 13.04 and 26.31).
  // Q8 keeps one block (2.6x slower with two of half the rows), and d = 256
  // gains nothing (8q/4kv window 1024: 9.28 against 9.28 us).
  static constexpr bool H2 = (D > 256 || (D == 128 && sizeof(T) == 4)) && sizeof(T) != 1 &&
                             RB >= 2 && (RB / 2) % RPS == 0 && (RB / 2) % RPI == 0;
  using C = Cfg<D, GH, T, LPR, H2 ? RB / 2 : RB, NW, H2 ? 2 : 1>;
};

// Dynamic LDS layout shared by host (size) and device (offsets), in floats.
struct Lds {
  int qs, cs, sn, knew, vnew, nw, pw, wm, wl, red, blk, misc, mrg, qw, psum, total;
  __host__ __device__ Lds(int D, int GH, int NW, int RB, int chunk, int page_shift, bool paged,
                          int merge) {
    const bool wide = D / 4 > 64;  // a q row spans more than one wave (d = 512)
    int o = 0;
    qs = o; o += GH * D;
    qw = o; o += wide ? D : 0;       // q norm weights
    // q rows' sums of squares, per 64 quads (padded: later regions are read
    // as 16-byte vectors)
    psum = o; o += wide ? (GH * (D / 256) + 3) / 4 * 4 : 0;
    cs = o; o += D / 2;
    sn = o; o += D / 2;
    knew = o; o += D;
    vnew = o; o += D;
    nw = o; o += D;                  // k norm weights
    pw = o; o += NW * RB * GH;
    wm = o; o += NW * GH;
    wl = o; o += NW * GH;
    red = o; o += NW * GH * D;       // per-wave o
    blk = o; o += paged ? ((chunk >> page_shift) + 2) : 0;
    misc = o; o += 8;                // block claim counter, merge flag
    mrg = o; o += merge;             // in-launch merge: chunk statistics
    total = o;
  }
};


// Workgroup barrier that orders LDS accesses only.  __syncthreads() also
// waits for every outstanding global load and store of the thread
// (s_waitcnt vmcnt(0)), which would stall the prologue on the K/V blocks
// already in flight.  No global data crosses workgroups inside a launch
// (the combine is a separate kernel).
// s_waitcnt vmcnt(N) alone (expcnt and lgkmcnt at their maxima; gfx9
// encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (((N >> 4) & 3) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// RMS norms of the step's fresh vectors (forward.h:554, 562-563):
// y = (x * 1/sqrt(mean(x^2) + eps)) * w (rmsnorm, include/molot/norm.h:9-28).
//
// q, in registers before it is staged: thread i of the prologue holds the
// float4 i of the GH q rows, so each row is D/4 aligned lanes of a wave and
// its sum of squares a group sum, with no LDS round trip and no barrier.
template <int D, int QPT>
__device__ __forceinline__ void q_norm_regs(const AttnArgs& a, f32x4 (&qv)[QPT],
                                            const f32x4 (&qw)[QPT], int dh) {
  static_assert(D / 4 <= 64 && 64 % (D / 4) == 0, "a q row within one wave");
#pragma unroll
  for (int u = 0; u < QPT; ++u) {
    float ss = qv[u][0] * qv[u][0];
    ss = fmaf(qv[u][1], qv[u][1], ss);
    ss = fmaf(qv[u][2], qv[u][2], ss);
    ss = fmaf(qv[u][3], qv[u][3], ss);
    const float inv = 1.0f / sqrtf(group_sum<D / 4>(ss) / (float)dh + a.eps);
#pragma unroll
    for (int e = 0; e < 4; ++e) qv[u][e] = qv[u][e] * inv * qw[u][e];
  }
}

// k and v of the new token, in the workgroup that appends it: the waves'
// partial sums of squares go to LDS before the prologue's barrier (k: one
// element per thread; v: all nkv*D values of v_new, see v_norm_load), and
// the threads that rotate k and round v after that barrier scale them:
// k by 1/sqrt(mean(k^2) + eps) and its weights (staged in LDS), v by the RMS
// of all of v_new without weights (rmsnorm_plain, norm.h:82-96).
__device__ __forceinline__ void k_norm_share(int w, int lane, float ss, float* ksum) {
  ss = group_sum<64>(ss);
  if (lane == 0) ksum[w] = ss;
}

struct NewNorms {
  float kinv, vinv;
  __device__ __forceinline__ void apply(const AttnArgs& a, const float* kw, int j, int half,
                                        float& k0, float& k1, float& v0, float& v1) const {
    if (a.k_norm) {
      k0 = k0 * kinv * kw[j];
      k1 = k1 * kinv * kw[j + half];
    }
    if (a.v_norm) {
      v0 *= vinv;
      v1 *= vinv;
    }
  }
};

template <int D, int NW>
__device__ __forceinline__ NewNorms new_norms(const AttnArgs& a, const float* ksum,
                                              const float* vsum, int dh) {
  NewNorms r{1.f, 1.f};
  if (a.k_norm) {
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < NW; ++k) ss += ksum[k];
    r.kinv = 1.0f / sqrtf(ss / (float)dh + a.eps);
  }
  if (a.v_norm) {
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < NW; ++k) ss += vsum[k];
    r.vinv = 1.0f / sqrtf(ss / (float)(a.nkv * dh) + a.eps);
  }
  return r;
}

// The joint v norm needs all nkv*D values of the sequence's v_new.  Their
// loads are issued in the prologue before any K/V row (loads retire in
// order, so the sum below does not wait for the stream's first block), up
// to kVnPT per thread; the rest, if any, are summed by a plain loop.
constexpr int kVnPT = 8;

template <int D, int NT>
__device__ __forceinline__ void v_norm_load(const AttnArgs& a, int b, int tid, float (&vq)[kVnPT],
                                            int dh) {
  const float* vx = a.v_new + (int64_t)b * a.nkv * dh;
  const int nv = a.nkv * dh;
#pragma unroll
  for (int u = 0; u < kVnPT; ++u) vq[u] = tid + u * NT < nv ? vx[tid + u * NT] : 0.f;
}

// The wave's sum of squares of its threads' shares into vsum[w].
template <int D, int NT>
__device__ __forceinline__ void v_norm_share(const AttnArgs& a, int b, int tid, int w, int lane,
                                             const float (&vq)[kVnPT], float* vsum, int dh) {
  float ss = 0.f;
#pragma unroll
  for (int u = 0; u < kVnPT; ++u) ss = fmaf(vq[u], vq[u], ss);
  const float* vx = a.v_new + (int64_t)b * a.nkv * dh;
  for (int j = tid + kVnPT * NT; j < a.nkv * dh; j += NT) ss = fmaf(vx[j], vx[j], ss);
  ss = group_sum<64>(ss);
  if (lane == 0) vsum[w] = ss;
}

// The workgroup's chunk partial from its waves' partials in LDS: running
// max wm[w*GH + g], sum wl[w*GH + g] and unnormalised o red[w*RS + g*D + d]
// of wave w (waves without rows hold max -inf).  A single-chunk problem
// writes O = o / l (and, with ROPE, the rotated q from qs) directly;
// otherwise (o, max, sum) goes to the workspace for combine_kernel.
// ---------------------------------------------------------------------------
// In-launch merge of the split-K chunk partials.
//
// Workgroup i runs on XCD i % 8 (the dispatch order of MI355X in its
// single-partition mode, checked once per device by xcd_map_ok() before the
// library relies on it), and the launch places every chunk of a slot on the
// same XCD.  The slot's partials therefore meet in one L2, the coherence
// point of that XCD's CUs, and the hand-off needs no cache writeback:
//   - each workgroup stores its partial (plain stores, which write through
//     the CU's L1 into the L2), waits until the L2 has acknowledged them
//     (a workgroup-scope release fence, s_waitcnt vmcnt(0), in every thread,
//     then a barrier) and adds one arrival to the slot's 64-bit arrival word
//     (a device-scope atomic, coherent across the XCDs);
//   - the arrival adds 1 + x*2^13 + x^2*2^29 for its XCD x = XCC_ID: the
//     word counts the arrivals (bits 0-12), and sums x (bits 13-28) and x^2
//     (bits 29-63).  The workgroup whose add completes the count arrived
//     last: every other chunk's stores were acknowledged before its arrival.
//     It resets the word to 0 for the next launch.  All nch chunks ran on
//     its own XCD m exactly when the sums are nch*m and nch*m^2 (the
//     variance of the XCDs is then 0), checked from the atomic's own
//     return value, so a violated dispatch assumption can never be read
//     from a stale record: the output is then NaN, never a stale merge;
//   - it reads the partials back with loads that miss the L1 (cache policy
//     sc0), so they come from the L2, merges them with log-sum-exp weights
//     as combine_kernel does and writes O and, with ROPE, the rotated q
//     (every workgroup of the slot has read q by the time it arrives).
// No workgroup waits for another: nothing spins, and a launch's arrivals
// are exactly its slots' chunk counts, so the words are back at zero when
// it ends (they are zeroed when the workspace is allocated).
constexpr int kArriveCountBits = 13;  // arrivals of a slot: at most kMergeMaxChunks
constexpr int kArriveSumBits = 16;    // sum of XCC_ID over the arrivals (<= 7 * 4096)
__device__ __forceinline__ unsigned long long arrive_word(int x) {
  const unsigned long long ux = (unsigned long long)x;
  return 1ull | (ux << kArriveCountBits) | ((ux * ux) << (kArriveCountBits + kArriveSumBits));
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t l2_rsrc(const float* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, 0x7FFFFFFF, 0x00020000);
}
// Loads at a byte offset of a resource, missing the L1 (cache policy sc0).
__device__ __forceinline__ f32x4 ld_l2x4(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 1));
}

__device__ __forceinline__ float2 ld_l2x2(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 1));
}

// XCD (accelerator complex) of the calling wave: hardware register XCC_ID.
__device__ __forceinline__ int xcc_id() {
  return (int)(__builtin_amdgcn_s_getreg((20) | (0 << 6) | (3 << 11)) & 15);
}

// Output element pr of a head group's GH x D tile (head g = pr / D, element
// j = pr % D) in the caller's [..][dh] rows: its index from qrow0's row, or
// -1 for the padding (j >= dh) of a padded launch.
__device__ __forceinline__ int64_t out_index(int64_t qrow0, int pr, int D, int dh) {
  const int g = pr / D, j = pr - g * D;
  return j < dh ? (qrow0 + g) * dh + j : -1;
}

// Stores float4 quad q (elements 4q .. 4q+3 of the GH x D tile) of a head
// group's output; dh is even, so a quad is whole or half inside a row.
__device__ __forceinline__ void store_quad(float* o, int64_t qrow0, int q, f32x4 v, int D, int dh) {
  const int64_t i0 = out_index(qrow0, 4 * q, D, dh);
  if (i0 < 0) return;
  if (dh == D || 4 * q % D + 4 <= dh) {
    if ((i0 & 3) == 0) {
      *reinterpret_cast<f32x4*>(o + i0) = v;
    } else {  // dh % 4 == 2: an 8-byte aligned row start
      *reinterpret_cast<float2*>(o + i0) = float2{v[0], v[1]};
      *reinterpret_cast<float2*>(o + i0 + 2) = float2{v[2], v[3]};
    }
  } else {
    *reinterpret_cast<float2*>(o + i0) = float2{v[0], v[1]};
  }
}

constexpr int kMergeMaxChunks = 4096;  // chunks of a slot merged in the launch
static_assert(kMergeMaxChunks < (1 << kArriveCountBits) &&
                  7 * kMergeMaxChunks < (1 << kArriveSumBits) &&
                  49ull * kMergeMaxChunks < (1ull << (64 - kArriveCountBits - kArriveSumBits)),
              "arrival word fields");
constexpr int kMergeAutoSpan = 8192;   // rows from which the default merges in the launch
constexpr int kMergeMaxPhases = 64;    // threads per float4 quad of the output (NT / quads)
constexpr int kMergeRound = 8;         // chunks per thread whose loads are in flight together

// LDS floats of the in-launch merge's phase statistics (Lds::mrg, LdsM::mrg).
__host__ __device__ constexpr int merge_lds_floats(int gh) { return 2 * kMergeMaxPhases * gh; }

// The merge of the workgroup that completes a slot.  Thread t owns float4
// quad q = t % QV of the slot's output (head g = 4q / D) in phase
// ph = t / QV; it folds chunks ph, ph + PH, ph + 2*PH, ... with a running
// log-sum-exp, kMergeRound chunks' loads in flight at a time and only the
// chunks that exist loaded.  The PH phases of a quad then merge once
// through LDS: their (max, sum) per head at mst, their o at mred.  Wave 0
// alone reads the chunks' XCD records (lane c: chunks c, c + 64, ...): with
// a record load per chunk in every thread the merge took 0.4 us longer
// (32q/8kv/d128 fp32, n = 16385).
// RED: floats of LDS at mred (the phase sums: PH*P floats).
template <int D, int GH, int NW, int NT, bool ROPE, int RED, int QSTR = D>
__device__ __forceinline__ void arrive_and_merge(const AttnArgs& a, int64_t slot, int nch,
                                                 int64_t qrow0, const float* qs, float* mst,
                                                 float* mred, int* flag, int tid, int lane,
                                                 int dh) {
  constexpr int P = GH * D;
  // this thread's partial stores are acknowledged by the L2 (vmcnt(0):
  // outside threadgroup-split mode the workgroup-scope release fence alone
  // need not wait for them)
  wait_vmcnt<0>();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  lds_barrier();
  if (tid == 0) {
    const int x = xcc_id();
    const unsigned long long tot = atomicAdd(a.ctr + slot, arrive_word(x)) + arrive_word(x);
    const bool last = (int)(tot & ((1ull << kArriveCountBits) - 1)) == nch;
    if (last) atomicExch(a.ctr + slot, 0ull);  // ready for the next launch
    const unsigned long long n64 = (unsigned long long)nch, x64 = (unsigned long long)x;
    const bool one_xcd = ((tot >> kArriveCountBits) & ((1ull << kArriveSumBits) - 1)) == n64 * x64 &&
                         (tot >> (kArriveCountBits + kArriveSumBits)) == n64 * x64 * x64;
    flag[0] = last;
    flag[1] = last && !one_xcd;  // a chunk of the slot ran on another XCD
  }
  lds_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  if (!flag[0]) return;  // uniform over the workgroup

  constexpr int QV = P / 4;                     // float4 quads of the slot's output
  // phases per quad: as many as the threads allow and the phase sums' LDS holds
  constexpr int PH0 = NT >= QV ? NT / QV : 1;
  constexpr int PH = PH0 * P <= RED ? PH0 : (RED / P > 1 ? RED / P : 1);
  constexpr int NQ = NT >= QV ? 1 : (QV + NT - 1) / NT;  // quads per thread
  static_assert(P % 4 == 0 && D % 4 == 0, "float4 quads");
  static_assert(PH <= kMergeMaxPhases, "phase statistics fit their LDS");
  const int ph = NT >= QV ? tid / QV : 0;
  const bool act = ph < PH;  // threads past PH * QV idle (NT not a multiple of QV)
  const __amdgpu_buffer_rsrc_t ro = l2_rsrc(a.part_o + slot * a.nchunks * P);
  const __amdgpu_buffer_rsrc_t rm = l2_rsrc(a.part_ml + slot * a.nchunks * (GH * 2));
  int qd[NQ], g[NQ];
  float m[NQ], l[NQ];
  f32x4 o[NQ];
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    qd[i] = NT >= QV ? tid % QV : min(tid + i * NT, QV - 1);
    g[i] = 4 * qd[i] / D;
    m[i] = -INFINITY;
    l[i] = 0.f;
    o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  for (int c0 = act ? ph : nch; c0 < nch; c0 += PH * kMergeRound) {
    float2 st[NQ][kMergeRound];
    f32x4 ov[NQ][kMergeRound];
#pragma unroll
    for (int u = 0; u < kMergeRound; ++u) {
      const int cc = c0 + PH * u;
#pragma unroll
      for (int i = 0; i < NQ; ++i) {
        if (cc < nch) {
          st[i][u] = ld_l2x2(rm, 8 * (cc * GH + g[i]));
          ov[i][u] = ld_l2x4(ro, 16 * (cc * QV + qd[i]));
        } else {
          st[i][u] = float2{-INFINITY, 0.f};
          ov[i][u] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      float mn = m[i];
#pragma unroll
      for (int u = 0; u < kMergeRound; ++u) mn = fmaxf(mn, st[i][u].x);
      const float al = softmax_exp(m[i] - mn);  // m = -inf on the first round: 0
      l[i] *= al;
      o[i] *= al;
#pragma unroll
      for (int u = 0; u < kMergeRound; ++u) {
        const float wc = softmax_exp(st[i][u].x - mn);  // absent chunks: e^-inf = 0
        l[i] = fmaf(wc, st[i][u].y, l[i]);
        o[i] += wc * ov[i][u];
      }
      m[i] = mn;
    }
  }
  // The hand-off above holds only if every chunk of the slot ran on this
  // XCD (one L2): otherwise the output is NaN, never a silently stale merge.
  const float bad = flag[1] ? __builtin_nanf("") : 0.f;
  if constexpr (PH > 1) {
    // a phase's (max, sum) is the same for every quad of a head: the
    // thread holding the head's first quad publishes it
    if (act) {
      reinterpret_cast<f32x4*>(mred)[ph * QV + qd[0]] = o[0];
      if ((4 * qd[0]) % D == 0) {
        mst[(ph * GH + g[0]) * 2] = m[0];
        mst[(ph * GH + g[0]) * 2 + 1] = l[0];
      }
    }
    lds_barrier();
    if (tid < QV) {
      float M = -INFINITY;
#pragma unroll
      for (int q2 = 0; q2 < PH; ++q2) M = fmaxf(M, mst[(q2 * GH + g[0]) * 2]);
      float Ls = 0.f;
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q2 = 0; q2 < PH; ++q2) {
        const float wq = softmax_exp(mst[(q2 * GH + g[0]) * 2] - M);  // phases with no chunk: 0
        Ls = fmaf(wq, mst[(q2 * GH + g[0]) * 2 + 1], Ls);
        acc += wq * reinterpret_cast<const f32x4*>(mred)[q2 * QV + tid];
      }
      store_quad(a.o, qrow0, tid, acc / Ls + bad, D, dh);
    }
  } else {
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int q4 = NT >= QV ? tid : tid + i * NT;
      if (act && q4 < QV) store_quad(a.o, qrow0, q4, o[i] / l[i] + bad, D, dh);
    }
  }
  if constexpr (ROPE) {
    if (a.q_out)
      for (int i = tid; i < P; i += NT) {
        const int64_t oi = out_index(qrow0, i, D, dh);
        if (oi >= 0) a.q_out[oi] = qs[(i / D) * QSTR + i % D];
      }
  }
}

template <int D, int GH, int NW, int NT, bool ROPE, int RED, bool XSW = false, int QSTR = D>
__device__ __forceinline__ void finish_chunk(const AttnArgs& a, const float* wm, const float* wl,
                                             const float* red, int RS, const float* qs, int tid,
                                             int lane, bool split, int64_t slot, int c,
                                             int64_t qrow0, int nch, float* mst, float* mred,
                                             int* flag, int dh) {
  constexpr int P = GH * D;
  // Every thread derives the chunk partial of its own output pairs from the
  // wave partials (wave weights e^(m_w - M); waves without rows weigh
  // e^-inf = 0).  Pairs: tid % Q + i*Q, i < PP; phase ph = tid / P.
  constexpr int PP = (P + NT - 1) / NT, Q = P < NT ? P : NT;
  const int ph = PP == 1 ? tid / P : 0;
  int pr_[PP], g_[PP];
  bool pv_[PP];
  float po[PP], pm[PP], pl[PP];
  // The 64 pairs of a wave lie in one head (D is a multiple of 64), so the
  // wave weights are wave-uniform: lane ww < NW computes wave ww's weight,
  // DPP/shuffle reductions give the chunk max and sum, and the weights reach
  // every lane through readlane.
  static_assert(D % 64 == 0 && NW <= 64, "wave-uniform head per 64 pairs");
#pragma unroll
  for (int i = 0; i < PP; ++i) {
    pr_[i] = tid % Q + i * Q;
    pv_[i] = pr_[i] < P;
    g_[i] = pv_[i] ? pr_[i] / D : 0;
    const int g = __builtin_amdgcn_readfirstlane(g_[i]);
    const float mw_l = lane < NW ? wm[lane * GH + g] : -INFINITY;
    const float m = group_max<NW <= 16 ? 16 : 64>(mw_l);  // lanes >= NW hold -inf
    // waves without rows weigh 0 (also when no wave of the chunk has one)
    const float e_l = lane < NW && mw_l != -INFINITY ? softmax_exp(mw_l - m) : 0.f;
    const float l = group_sum<NW <= 16 ? 16 : 64>(lane < NW ? e_l * wl[lane * GH + g] : 0.f);
    float o = 0.f;
    // XSW: head g's element j at g*D + (j ^ 4*(g % 8)) (the matrix-core
    // kernel's conflict-free layout)
    const int ri =
        !pv_[i] ? 0 : XSW ? g_[i] * D + ((pr_[i] - g_[i] * D) ^ (4 * (g_[i] & 7))) : pr_[i];
#pragma unroll
    for (int ww = 0; ww < NW; ++ww)
      o = fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(e_l), ww)),
               red[ww * RS + ri], o);
    po[i] = o;
    pm[i] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(m)));
    pl[i] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(l)));
  }
  const bool lead = ph == 0;  // phase 0 threads own the chunk partial's outputs
  if (!split) {
#pragma unroll
    for (int i = 0; i < PP; ++i) {
      const int64_t oi = lead && pv_[i] ? out_index(qrow0, pr_[i], D, dh) : -1;
      if (oi >= 0) a.o[oi] = po[i] / pl[i];
    }
    if constexpr (ROPE) {
      if (a.q_out)
        for (int i = tid; i < P; i += NT) {
          const int64_t oi = out_index(qrow0, i, D, dh);
          if (oi >= 0) a.q_out[oi] = qs[(i / D) * QSTR + i % D];
        }
    }
    return;
  }

  // ---- 5. the chunk partial for the combine kernel ----
  // Plain stores: the combine kernel runs after this one on the same stream,
  // so the kernel boundary orders them; no flag, counter or cleared memory
  // is needed between the two launches.
  float* po_s = a.part_o + (slot * a.nchunks + c) * P;
  float* pml_s = a.part_ml + (slot * a.nchunks + c) * (GH * 2);
#pragma unroll
  for (int i = 0; i < PP; ++i) {
    if (!(lead && pv_[i])) continue;
    po_s[pr_[i]] = po[i];
    if (pr_[i] - g_[i] * D == 0) {
      pml_s[2 * g_[i]] = pm[i];
      pml_s[2 * g_[i] + 1] = pl[i];
    }
  }
  if (a.ctr) {  // in-launch merge: the workgroup completing the slot merges it
    arrive_and_merge<D, GH, NW, NT, ROPE, RED, QSTR>(a, slot, nch, qrow0, qs, mst, mred, flag, tid,
                                               lane, dh);
    return;
  }
  if constexpr (ROPE) {  // the rotated q leaves through the combine kernel
    if (c == 0 && a.q_out)
      for (int i = tid; i < P; i += NT) a.qrot[slot * P + i] = qs[(i / D) * QSTR + i % D];
  }
}

// A sequence of a batch whose window leaves no cache row attended, in a
// launch that appends nothing (a layer reading another layer's KV,
// forward.h:578-585): its q rows are still normed and rotated in place, as
// forward.h:554-558 does before every attention call, and its o is 0
// (attn.h:162 with no rows).  The whole workgroup takes this path; nothing
// else is in flight, so plain workgroup barriers are free here.  Same
// arithmetic as rope_append_kernel: (x * 1/sqrt(mean(x^2) + eps)) * w, then
// the NEOX rotation by the fp32 angle pos * inv_freq[j] (sine and cosine in
// double, rounded).
template <int NT>
__device__ void empty_range_q(const AttnArgs& a, int64_t qrow0, int gh, int dh, int pos,
                              float* sh) {
  const int tid = threadIdx.x, half = dh / 2;
  const bool rot = a.inv_freq != nullptr;
  for (int g = 0; g < gh; ++g) {
    const float* x = a.q + (qrow0 + g) * dh;
    float* y = a.q_out + (qrow0 + g) * dh;
    float inv = 1.f;
    if (a.q_norm) {  // uniform
      float ss = 0.f;
      for (int j = tid; j < dh; j += NT) ss = fmaf(x[j], x[j], ss);
      inv = 1.0f / sqrtf(block_sum(ss, sh) / (float)dh + a.eps);
    }
    for (int j = tid; j < half; j += NT) {
      float x0 = x[j], x1 = x[j + half];
      if (a.q_norm) {
        x0 = x0 * inv * a.q_norm[j];
        x1 = x1 * inv * a.q_norm[j + half];
      }
      if (rot) {
        const float ang = (float)pos * a.inv_freq[j];
        double sd, cd;
        sincos((double)ang, &sd, &cd);
        const float c = (float)cd, sn = (float)sd;
        y[j] = x0 * c - x1 * sn;
        y[j + half] = x0 * sn + x1 * c;
      } else {
        y[j] = x0;
        y[j + half] = x1;
      }
    }
  }
}

template <int D, int GH, typename T, bool PAGED, bool ROPE, bool PAD, typename C>
__global__ __launch_bounds__(C::NT) void attn_kernel(AttnArgs a) {
  using V16 = typename KVT<T>::vec;
  constexpr int VW = C::VW, LPR = C::LPR, NV = C::NV, EPL = C::EPL, RPS = C::RPS;
  constexpr int LPR2 = C::LPR2, RPI = C::RPI, RB = C::RB, KS = C::KS, VS = C::VS;
  constexpr int NV2 = C::NV2, AW = C::AW;
  constexpr int NW = C::NW, NT = C::NT, P = C::P;

  extern __shared__ float smem[];
  const Lds L(D, GH, NW, RB, a.chunk, a.page_shift, PAGED, a.mrg);
  float* qs = smem + L.qs;
  float* knew = smem + L.knew;
  float* vnew = smem + L.vnew;
  int* misc = reinterpret_cast<int*>(smem + L.misc);

  // PAD: heads of DH < D elements, run as D with q zero-padded (load_pad)
  const int DH = PAD ? a.dh : D;
  // Q8 (D = 256; the matrix-core kernel takes 64 and 128): 16 codes per
  // 16-byte load, an fp32 scale per K and V row, applied to the row's score
  // and to its probability in PV
  constexpr bool Q8 = sizeof(T) == 1;
  const int G = a.nq / a.nkv;
  const int nsub = G / GH;
  // chunk slot z (chunk c = nch - 1 - z, below), (KV head, subgroup) index
  // hs and sequence b of this workgroup; X (KV head, subgroup) pairs per
  // sequence
  const int X = a.nkv * nsub;
  int z = blockIdx.z, hs = blockIdx.x, b = blockIdx.y;
  if (a.xmap) {  // slot id % 8 runs on XCD id % 8 (launch_pair); padding ids exit
    const int s8 = (int)(blockIdx.x & 7);
    if (s8 >= a.slots) return;
    z = (int)(blockIdx.x >> 3);
    hs = s8 % X;
    b = s8 / X;
  } else if (a.chunk_fast) {  // Q8: a chunk's heads on one XCD, as attn_mfma_kernel
    const int k = (int)(blockIdx.x >> 3);
    const int pi = (k / X) * 8 + (int)(blockIdx.x & 7);  // padded ids (z >= nchunks) exit below
    z = pi / a.nseq;
    b = pi - z * a.nseq;
    hs = k % X;
  }
  const int sub = hs % nsub;
  const int h = hs / nsub;
  const int hq0 = h * G + sub * GH;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform

  int n = a.n, t0 = a.t0, pos = a.pos;
  // per-sequence ranges in contiguous chunks: a paged batch, or prefill rows
  bool perseq = PAGED;
  if constexpr (!ROPE) perseq = PAGED || a.pf;  // uniform
  if (perseq) {
    if (!ROPE && a.pf) {
      pos = a.pos + b;
      n = min(pos + 1, a.n);
    } else {
      n = a.seq_lens[b];
      pos = a.pos_arr ? a.pos_arr[b] : n - 1;
    }
    t0 = (a.window > 0 && pos - a.window + 1 > 0) ? pos - a.window + 1 : 0;
    if (t0 > n) t0 = n;
  }
  // Chunks tile the cache rows [t0, cend); a fused step's new token (slot
  // n-1) is not read from the cache but folded into the last chunk.
  const bool fold = ROPE && a.fold;  // this launch appends and folds in the new token
  const int cend = fold ? n - 1 : n;
  int nch = a.nchunks;
  if (perseq) {
    const int span = cend - t0;
    nch = span > 0 ? (span + a.chunk - 1) / a.chunk : (fold ? 1 : 0);
    if (nch > a.nchunks) nch = a.nchunks;
  }
  if (z >= nch) {  // whole workgroup: chunk past this sequence's end (never arrives)
    if (z == 0) {  // empty attended range: o = 0 (include/molot/attn.h:162 with no rows)
      for (int i = tid; i < GH * DH; i += NT) a.o[((int64_t)b * a.nq + hq0) * DH + i] = 0.f;
      if (ROPE && !fold && a.q_out)  // nothing appended: q still leaves normed and rotated
        empty_range_q<NT>(a, (int64_t)b * a.nq + hq0, GH, DH, pos, smem);
    }
    return;
  }
  // Chunks in reverse: the last one, which holds the new token (and with it
  // the append, the fold and any norms of k and v), is dispatched first.
  const int c = nch - 1 - z;
  const int tb = t0 + c * a.chunk;
  const int cntg = max(0, min(a.chunk, cend - tb));  // rows read from the cache
  const bool is_new = fold && c == nch - 1;          // this chunk folds in the new token
  const bool split = nch > 1;
  const int64_t slot = (int64_t)b * X + hs;

  const T* __restrict__ Kb = reinterpret_cast<const T*>(a.k);
  const T* __restrict__ Vb = reinterpret_cast<const T*>(a.v);
  const int64_t hoff = (int64_t)h * a.head_stride;
  const int64_t qrow0 = (int64_t)b * a.nq + hq0;

  // ---- 1. prologue ----
  if constexpr (PAGED) {
    int32_t* sblk_w = reinterpret_cast<int32_t*>(smem + L.blk);
    // the chunk's pages (at least the one holding row tb, which exists:
    // tb <= n-1, so the clamped loads of an empty chunk stay in bounds)
    const int p0 = tb >> a.page_shift;
    const int p1 = max(p0, (tb + cntg - 1) >> a.page_shift);
    for (int i = tid; i <= p1 - p0; i += NT)
      sblk_w[i] = a.block_table[(int64_t)b * a.max_blocks + p0 + i];
    lds_barrier();
  }
  const int32_t* sblk = reinterpret_cast<const int32_t*>(smem + L.blk);
  auto row_ptr = [&](const T* base, int t) -> const T* {
    if constexpr (PAGED) {
      const int pg = (t >> a.page_shift) - (tb >> a.page_shift);
      return base + (int64_t)sblk[pg] * a.block_stride + hoff +
             (int64_t)(t & ((1 << a.page_shift) - 1)) * a.tok_stride;
    } else {
      return base + (int64_t)t * a.tok_stride + hoff;
    }
  };
  // Q8: the fp32 scale of row t of head h
  auto sc_ptr = [&](const T* base, int t) -> const float* {
    const char* p = reinterpret_cast<const char*>(base) + a.sc_off + h * a.sc_head;
    if constexpr (PAGED) {
      const int pg = (t >> a.page_shift) - (tb >> a.page_shift);
      return reinterpret_cast<const float*>(p + (int64_t)sblk[pg] * a.block_stride) +
             (t & ((1 << a.page_shift) - 1));
    } else {
      return reinterpret_cast<const float*>(p + (int64_t)t * a.tok_stride);
    }
  };
  const int s = lane % LPR;    // scores: lane within a K row group
  const int rr = lane / LPR;   // scores: row of the group within a K step
  const int cs = lane % LPR2;  // PV: columns cs*VW .. cs*VW+VW-1
  const int rs = lane / LPR2;  // PV: row within a V step
  V16 kA[KS][NV], vA[VS][NV2], kB[KS][NV], vB[VS][NV2];
  float ksA[KS], vsA[VS], ksB[KS], vsB[VS];  // Q8 row scales (unused otherwise)
  // Every wave issues the same sequence of global loads on every path: the
  // compiler counts outstanding loads per path and, where paths merge with
  // different counts, waits for all of them.  Rows past the end (a partial
  // block, or a block past the last) load the last row instead (the first
  // of an empty range): no branch around the loads, no extra HBM traffic
  // (lines of a row already read), and a probability of e^-inf = 0 where
  // they are scored at all.
  // Row mapping.  Paged: the chunk's rows [tb, tb + cntg), in order.  A
  // contiguous cache: the chunk's local row lr lies in its (lr/32)-th 32-row
  // group, the range's group c + (lr/32)*nch (groups dealt round robin, so
  // the launch's workgroups read neighbouring rows at any moment; blocks of
  // RB rows never straddle a group).
  static_assert(32 % RB == 0, "blocks within 32-row groups");
  const int rlim = perseq ? cntg : cend - t0;  // rows of the chunk / of the whole range
  const int rfirst = perseq ? tb : t0;
  const int rmax = max(rlim - 1, 0);
  auto gmap = [&](int lr) -> int {  // local row -> row from rfirst
    return perseq ? lr : (c + (lr >> 5) * nch) * 32 + (lr & 31);
  };
  // Local rows of this chunk: its valid rows come first, so every block
  // below nblk starts with a valid row (a block of no valid rows would meet
  // m_run = -inf with a -inf score: e^(-inf - -inf) is NaN).  The chunk
  // holding the range's last group counts only that group's valid rows.
  int nrows = cntg;
  if (!perseq) {
    const int groups = (rlim + 31) / 32;
    nrows = 0;
    if (c < groups) {
      const int last = (groups - 1 - c) / nch;  // local index of the chunk's last group
      nrows = 32 * last + min(32, rlim - 32 * (c + last * nch));
    }
  }
  auto load_block = [&](V16 (&kr)[KS][NV], V16 (&vr)[VS][NV2], float (&ksr)[KS], float (&vsr)[VS],
                        int rbase) {
#pragma unroll
    for (int k = 0; k < KS; ++k) {
      const int t = rfirst + min(gmap(rbase + k * RPS + rr), rmax);
      const T* p = row_ptr(Kb, t);
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        if constexpr (PAD)
          kr[k][v] = load_pad(p, (v * LPR + s) * VW, DH);
        else
          kr[k][v] = load16(p + (v * LPR + s) * VW);
      }
      if constexpr (Q8) ksr[k] = *sc_ptr(Kb, t);
    }
#pragma unroll
    for (int k = 0; k < VS; ++k) {
      const int t = rfirst + min(gmap(rbase + k * RPI + rs), rmax);
      const T* p = row_ptr(Vb, t);
#pragma unroll
      for (int v2 = 0; v2 < NV2; ++v2) {
        if constexpr (PAD)
          vr[k][v2] = load_pad(p, (v2 * LPR2 + cs) * VW, DH);
        else
          vr[k][v2] = load16(p + (v2 * LPR2 + cs) * VW);
      }
      if constexpr (Q8) vsr[k] = *sc_ptr(Vb, t);
    }
  };
  const int nblk = (nrows + RB - 1) / RB;
  // The prologue's own global loads go first: loads retire in order, so
  // waiting for them does not also wait for the K/V blocks issued next.
  constexpr int QV = GH * D / 4;  // float4s of q of the group
  constexpr int QPT = (QV + NT - 1) / NT;
  // the fresh k and v rows: KPT elements a thread (two at d = 512 on 4 waves)
  constexpr int KPT = (D + NT - 1) / NT;
  static_assert(D / 2 <= NT, "one thread per rotation pair in the prologue");
  // a q row wider than a wave (d = 512): its norm sums through LDS (psum)
  constexpr bool QWIDE = D / 4 > 64;
  f32x4 qv[QPT];
  // A padded launch reads the q rows (and the q norm weights) at their
  // stored length DH, in two-element pieces, each selected to 0 past DH:
  // q's zero padding to D.
  auto row_quad = [&](const float* base, int i, int64_t stride) -> f32x4 {
    if constexpr (!PAD) {
      return reinterpret_cast<const f32x4*>(base)[i];
    } else {
      const int g = i / (D / 4), j = 4 * (i - g * (D / 4));
      const float* r = base + g * stride;
      const float2 lo = *reinterpret_cast<const float2*>(r + (j < DH ? j : 0));
      const float2 hi = *reinterpret_cast<const float2*>(r + (j + 2 < DH ? j + 2 : 0));
      return f32x4{j < DH ? lo.x : 0.f, j < DH ? lo.y : 0.f, j + 2 < DH ? hi.x : 0.f,
                   j + 2 < DH ? hi.y : 0.f};
    }
  };
#pragma unroll
  for (int u = 0; u < QPT; ++u) qv[u] = row_quad(a.q + qrow0 * DH, min(tid + u * NT, QV - 1), DH);
  float invf = 0.f, knv[KPT], vnv[KPT], kwv[KPT];
#pragma unroll
  for (int u = 0; u < KPT; ++u) knv[u] = vnv[u] = kwv[u] = 0.f;
  f32x4 qwt[QPT];  // q norm weights of this thread's q elements
  if constexpr (ROPE) {
    // every path issues these loads: a layer without RoPE (inv_freq NULL)
    // or without an append reads q in their place (nq >= nkv rows), unused
    const float* ivp = a.inv_freq ? a.inv_freq : a.q;
    const float* knp = fold ? a.k_new : a.q;
    const float* vnp = fold ? a.v_new : a.q;
    invf = ivp[min(tid, DH / 2 - 1)];
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int j = tid + u * NT;
      knv[u] = knp[((int64_t)b * a.nkv + h) * DH + min(j, DH - 1)];
      vnv[u] = vnp[((int64_t)b * a.nkv + h) * DH + min(j, DH - 1)];
      if (j >= DH) knv[u] = vnv[u] = 0.f;  // the padding of the new k and v rows
    }
    if (a.q_norm) {
#pragma unroll
      for (int u = 0; u < QPT; ++u)
        qwt[u] = row_quad(a.q_norm, min(tid + u * NT, QV - 1) % (D / 4), 0);
    }
    if (is_new && a.k_norm) {
#pragma unroll
      for (int u = 0; u < KPT; ++u) kwv[u] = a.k_norm[min(tid + u * NT, DH - 1)];
    }
  }
  float vq[kVnPT];
  const bool vn = ROPE && is_new && a.v_norm;  // uniform over the workgroup
  if (vn) v_norm_load<D, NT>(a, b, tid, vq, DH);
  // each wave's first NBUF blocks: w (and w + NW); the rest are claimed
  int bA = w, bB = w + NW;
  load_block(kA, vA, ksA, vsA, bA * RB);
  if constexpr (C::NBUF == 2) load_block(kB, vB, ksB, vsB, bB * RB);
  if (tid == 0) {
    misc[0] = C::NBUF * NW;  // next block to claim
  }
  if constexpr (ROPE) {
    if (a.q_norm) {
      if constexpr (!QWIDE) {
        q_norm_regs<D, QPT>(a, qv, qwt, DH);
      } else {
        // 64 consecutive quads (one wave's share of a u) lie in one row:
        // their sum of squares to psum[row][part]; the weights to qw.  The
        // rotation pass below applies the norm.
#pragma unroll
        for (int u = 0; u < QPT; ++u) {
          const int i = tid + u * NT;
          if (i < QV) {  // uniform over the wave: QV is a multiple of 64
            float ss = qv[u][0] * qv[u][0];
            ss = fmaf(qv[u][1], qv[u][1], ss);
            ss = fmaf(qv[u][2], qv[u][2], ss);
            ss = fmaf(qv[u][3], qv[u][3], ss);
            ss = group_sum<64>(ss);
            if (lane == 0) smem[L.psum + i / 64] = ss;
            if (i < D / 4) reinterpret_cast<f32x4*>(smem + L.qw)[i] = qwt[u];
          }
        }
      }
    }
  }
#pragma unroll
  for (int u = 0; u < QPT; ++u) {
    const int i = tid + u * NT;
    if (i < QV) reinterpret_cast<f32x4*>(qs)[i] = qv[u];
  }
  if constexpr (ROPE) {
    float* csn = smem + L.cs;
    float* sn = smem + L.sn;
    const bool rot = a.inv_freq != nullptr;  // uniform: no RoPE on a NoPE layer
    if (rot && tid < DH / 2) {
      const float ang = (float)pos * invf;
      double sd, cd;
      sincos((double)ang, &sd, &cd);
      csn[tid] = (float)cd;
      sn[tid] = (float)sd;
    }
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int j = tid + u * NT;
      if (j < D) {
        if (is_new) {
          knew[j] = knv[u];
          vnew[j] = vnv[u];
        }
        smem[L.nw + j] = kwv[u];
      }
    }
    if (vn) v_norm_share<D, NT>(a, b, tid, w, lane, vq, smem + L.wl, DH);
    if (is_new && a.k_norm) {
      float ss = 0.f;
#pragma unroll
      for (int u = 0; u < KPT; ++u) ss = fmaf(knv[u], knv[u], ss);  // 0 past D
      k_norm_share(w, lane, ss, smem + L.wm);
    }
    lds_barrier();
    // NEOX pairs (j, j + DH/2) of the stored head (attn.h:17-28); a q row
    // wider than a wave takes its norm here: (x * inv) * w, as q_norm_regs
    const int half = DH / 2;
    const bool qwn = QWIDE && a.q_norm;
    for (int i = tid; (rot || qwn) && i < GH * half; i += NT) {
      const int g = i / half, j = i - g * half;
      float x0 = qs[g * D + j], x1 = qs[g * D + j + half];
      if (qwn) {
        float ss = 0.f;
#pragma unroll
        for (int pt = 0; pt < D / 256; ++pt) ss += smem[L.psum + g * (D / 256) + pt];
        const float inv = 1.0f / sqrtf(ss / (float)DH + a.eps);
        x0 = x0 * inv * smem[L.qw + j];
        x1 = x1 * inv * smem[L.qw + j + half];
      }
      qs[g * D + j] = rot ? x0 * csn[j] - x1 * sn[j] : x0;
      qs[g * D + j + half] = rot ? x0 * sn[j] + x1 * csn[j] : x1;
    }
    if (is_new) {
      // the appended row as the cache will hold it: normed (as configured),
      // rotated k, k and v rounded to the cache type (stored into the cache
      // after the stream)
      const NewNorms nn = new_norms<D, NW>(a, smem + L.wm, smem + L.wl, DH);
      for (int j = tid; j < half; j += NT) {
        float k0 = knew[j], k1 = knew[j + half];
        float v0 = vnew[j], v1 = vnew[j + half];
        nn.apply(a, smem + L.nw, j, half, k0, k1, v0, v1);
        float r0 = rot ? k0 * csn[j] - k1 * sn[j] : k0;
        float r1 = rot ? k0 * sn[j] + k1 * csn[j] : k1;
        if constexpr (sizeof(T) == 2) {
          r0 = __uint_as_float((uint32_t)f32_to_bf16(r0) << 16);
          r1 = __uint_as_float((uint32_t)f32_to_bf16(r1) << 16);
          v0 = __uint_as_float((uint32_t)f32_to_bf16(v0) << 16);
          v1 = __uint_as_float((uint32_t)f32_to_bf16(v1) << 16);
        }
        knew[j] = r0;
        knew[j + half] = r1;
        vnew[j] = v0;
        vnew[j + half] = v1;
      }
    }
  }
  lds_barrier();

  // q registers: lane s of a K row group holds elements (v*LPR + s)*VW + e
  float qr[GH][EPL];
  // Base-2 scores: the dot products are scaled by scale*log2(e) as a whole
  // (one rounding per score, as the natural-units scale), not through a
  // pre-scaled q, whose per-element rounding perturbs q itself: with q
  // channels 1000x the rest that was 1.7e-5 normwise off float64, outside
  // the 1e-5 bar the score-scaled form meets.
  const float qsc = a.scale * kLog2e;
#pragma unroll
  for (int g = 0; g < GH; ++g)
#pragma unroll
    for (int v = 0; v < NV; ++v)
#pragma unroll
      for (int e4 = 0; e4 < VW; e4 += 4) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(qs + g * D + (v * LPR + s) * VW + e4);
        qr[g][v * VW + e4 + 0] = x[0];
        qr[g][v * VW + e4 + 1] = x[1];
        qr[g][v * VW + e4 + 2] = x[2];
        qr[g][v * VW + e4 + 3] = x[3];
      }

  // ---- 2. streaming blocks with a per-wave online softmax ----
  float* pw = smem + L.pw + w * RB * GH;
  float m_run[GH], l_run[GH], acc[GH][AW];
#pragma unroll
  for (int g = 0; g < GH; ++g) {
    m_run[g] = -INFINITY;
    l_run[g] = 0.f;
#pragma unroll
    for (int e = 0; e < AW; ++e) acc[g][e] = 0.f;
  }
  int next_fixed = w + C::NBUF * NW;  // fixed order: wave w takes blocks w, w+NW, w+2NW, ...
  auto claim = [&]() -> int {
    if (!a.dynamic) {
      const int v = next_fixed;
      next_fixed += NW;
      return v;
    }
    int v = 0;
    if (lane == 0) v = atomicAdd(&misc[0], 1);
    return __builtin_amdgcn_readfirstlane(v);
  };
  auto consume = [&](const V16 (&kr)[KS][NV], const V16 (&vr)[VS][NV2], const float (&ksr)[KS],
                     const float (&vsr)[VS], int rbase) {
    // scores of this lane group's rows
    float sc[KS][GH];
    float bmax[GH];
#pragma unroll
    for (int g = 0; g < GH; ++g) bmax[g] = -INFINITY;
#pragma unroll
    for (int k = 0; k < KS; ++k) {
      float d[GH];
#pragma unroll
      for (int g = 0; g < GH; ++g) d[g] = 0.f;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        float x[VW];
        KVT<T>::unpack(kr[k][v], x);
#pragma unroll
        for (int e = 0; e < VW; ++e)
#pragma unroll
          for (int g = 0; g < GH; ++g) d[g] = fmaf(qr[g][v * VW + e], x[e], d[g]);
      }
      const bool valid = rbase + k * RPS + rr < nrows;
#pragma unroll
      for (int g = 0; g < GH; ++g) {
        const float t = group_sum<LPR>(d[g]) * (Q8 ? qsc * ksr[k] : qsc);
        sc[k][g] = valid ? t : -INFINITY;
        bmax[g] = fmaxf(bmax[g], sc[k][g]);
      }
    }
    // The running max moves only when a score passes it by more than
    // kLazyMax (p <= 2^8 otherwise; o and l always share the max they were
    // formed with): most blocks skip the block max across the wave's row
    // groups and the rescale.
    bool grow = false;
#pragma unroll
    for (int g = 0; g < GH; ++g) grow |= bmax[g] > m_run[g] + kLazyMax;
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {  // wave-uniform
#pragma unroll
      for (int g = 0; g < GH; ++g) {
        auto bmax_off = [&](auto OFFC) {
          constexpr int off = decltype(OFFC)::value;
          if constexpr (off >= LPR) bmax[g] = max_xor<off>(bmax[g]);
        };
        bmax_off(std::integral_constant<int, 1>{});
        bmax_off(std::integral_constant<int, 2>{});
        bmax_off(std::integral_constant<int, 4>{});
        bmax_off(std::integral_constant<int, 8>{});
        bmax_off(std::integral_constant<int, 16>{});
        bmax_off(std::integral_constant<int, 32>{});
        const float mn = fmaxf(m_run[g], bmax[g]);
        const float alpha = exp2_hw(m_run[g] - mn);  // m_run = -inf -> 0
        m_run[g] = mn;
        l_run[g] *= alpha;
#pragma unroll
        for (int e = 0; e < AW; ++e) acc[g][e] *= alpha;
      }
    }
#pragma unroll
    for (int k = 0; k < KS; ++k) {
      if (s == 0) {
#pragma unroll
        for (int g = 0; g < GH; ++g) pw[(k * RPS + rr) * GH + g] = exp2_hw(sc[k][g] - m_run[g]);
      }
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int k = 0; k < VS; ++k) {
      float x[AW];
#pragma unroll
      for (int v2 = 0; v2 < NV2; ++v2) KVT<T>::unpack(vr[k][v2], x + v2 * VW);
      float p[GH];
#pragma unroll
      for (int g = 0; g < GH; ++g) p[g] = pw[(k * RPI + rs) * GH + g];
#pragma unroll
      for (int g = 0; g < GH; ++g) {
        l_run[g] += p[g];
        const float pv = Q8 ? p[g] * vsr[k] : p[g];  // Q8: codes times the V row's scale
#pragma unroll
        for (int e = 0; e < AW; ++e) acc[g][e] = fmaf(pv, x[e], acc[g][e]);
      }
    }
    __builtin_amdgcn_wave_barrier();
  };
  // Two buffers, A and B, alternate: a block's successor is claimed before
  // the block is consumed and loaded right after, so one block is always in
  // flight while the other is scored.  On the path that continues, every
  // load is unconditional (the exits drain the other buffer), so the
  // compiler waits only for the buffer about to be consumed.  Claims are
  // monotone: once a claim is past the end, every later one is too.
  // The explicit waits state what the compiler cannot always derive at the
  // rotated loop's header: the older buffer is complete while the younger
  // buffer's LB loads stay in flight.
  constexpr int LB = KS * NV + VS;  // loads per block
  if constexpr (C::NBUF == 1) {
    // one block in flight: score it, claim and load the next
    while (bA < nblk) {
      const int nx = claim();
      consume(kA, vA, ksA, vsA, bA * RB);
      bA = nx;
      if (bA < nblk) load_block(kA, vA, ksA, vsA, bA * RB);
    }
  } else if (bA < nblk) {
    if (bB >= nblk) {
      consume(kA, vA, ksA, vsA, bA * RB);
    } else {
      for (;;) {
        int nx = claim();
        wait_vmcnt<LB>();
        consume(kA, vA, ksA, vsA, bA * RB);
        if (nx >= nblk) {
          consume(kB, vB, ksB, vsB, bB * RB);
          break;
        }
        bA = nx;
        load_block(kA, vA, ksA, vsA, bA * RB);
        nx = claim();
        wait_vmcnt<LB>();
        consume(kB, vB, ksB, vsB, bB * RB);
        if (nx >= nblk) {
          consume(kA, vA, ksA, vsA, bA * RB);
          break;
        }
        bB = nx;
        load_block(kB, vB, ksB, vsB, bB * RB);
      }
    }
  }

  // ---- 3. the new token, folded in by wave 0 from LDS (its append to the
  // cache comes last, below) ----
  // Q8: wave 0 quantizes the k and v rows as the cache will hold them (the
  // reference quantizer, quant.h:34-50: s = absmax / 127, codes round(x/s))
  // and leaves code * s in LDS for the fold
  [[maybe_unused]] int kcode[Q8 ? D / 64 : 1], vcode[Q8 ? D / 64 : 1];
  [[maybe_unused]] float kscale = 0.f, vscale = 0.f;
  if constexpr (Q8) {
    if (is_new && w == 0) {
      constexpr int EPL = D / 64;
      float kx[EPL], vx[EPL];
      float ka = 0.f, va = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        kx[e] = knew[lane + 64 * e];
        vx[e] = vnew[lane + 64 * e];
        ka = fmaxf(ka, fabsf(kx[e]));
        va = fmaxf(va, fabsf(vx[e]));
      }
      kscale = q8_scale(group_max<64>(ka));
      vscale = q8_scale(group_max<64>(va));
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        kcode[e] = q8_code(kx[e], kscale);
        vcode[e] = q8_code(vx[e], vscale);
        knew[lane + 64 * e] = (float)kcode[e] * kscale;
        vnew[lane + 64 * e] = (float)vcode[e] * vscale;
      }
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");  // the fold reads other lanes' rows
    }
  }
  if (is_new && w == 0) {
    // LDS reads first, unconditional and vector-wide: the lanes of PV row 0
    // add the row's values, the others add 0 (a select per element, not a
    // branch around each read)
    const float one = rs == 0 ? 1.f : 0.f;
    float vx[AW];
#pragma unroll
    for (int v2 = 0; v2 < NV2; ++v2)
#pragma unroll
      for (int e4 = 0; e4 < VW; e4 += 4) {
        const f32x4 t = *reinterpret_cast<const f32x4*>(vnew + (v2 * LPR2 + cs) * VW + e4);
#pragma unroll
        for (int e = 0; e < 4; ++e) vx[v2 * VW + e4 + e] = t[e] * one;
      }
    float part[GH];
#pragma unroll
    for (int g = 0; g < GH; ++g) {
      part[g] = 0.f;
#pragma unroll
      for (int j = lane; j < D; j += 64) part[g] = fmaf(qs[g * D + j], knew[j], part[g]);
    }
#pragma unroll
    for (int g = 0; g < GH; ++g) {
      const float snew = wave_reduce<false>(part[g]) * qsc;
      const float mn = fmaxf(m_run[g], snew);
      const float alpha = exp2_hw(m_run[g] - mn);
      const float p = exp2_hw(snew - mn);
      m_run[g] = mn;
      l_run[g] = l_run[g] * alpha + p * one;
#pragma unroll
      for (int e = 0; e < AW; ++e) acc[g][e] = acc[g][e] * alpha + p * vx[e];
    }
  }

  // ---- 4. merge the waves ----
  // lanes LPR2 apart hold the same columns of other rows: sum them, in
  // ascending offsets
  auto merge_off = [&](auto OFFC) {
    constexpr int off = decltype(OFFC)::value;
    if constexpr (off >= LPR2) {
#pragma unroll
      for (int g = 0; g < GH; ++g) {
        l_run[g] = sum_xor<off>(l_run[g]);
#pragma unroll
        for (int e = 0; e < AW; ++e) acc[g][e] = sum_xor<off>(acc[g][e]);
      }
    }
  };
  merge_off(std::integral_constant<int, 1>{});
  merge_off(std::integral_constant<int, 2>{});
  merge_off(std::integral_constant<int, 4>{});
  merge_off(std::integral_constant<int, 8>{});
  merge_off(std::integral_constant<int, 16>{});
  merge_off(std::integral_constant<int, 32>{});
  float* wm = smem + L.wm;
  float* wl = smem + L.wl;
  float* red = smem + L.red;
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < GH; ++g) {
      wm[w * GH + g] = m_run[g] * kLn2;  // natural units for the merges
      wl[w * GH + g] = l_run[g];
    }
  }
  if (rs == 0) {
#pragma unroll
    for (int g = 0; g < GH; ++g)
#pragma unroll
      for (int v2 = 0; v2 < NV2; ++v2)
#pragma unroll
        for (int e = 0; e < VW; ++e)
          red[(w * GH + g) * D + (v2 * LPR2 + cs) * VW + e] = acc[g][v2 * VW + e];
  }
  lds_barrier();
  finish_chunk<D, GH, NW, NT, ROPE, NW * P>(a, wm, wl, red, P, qs, tid, lane, split, slot, c,
                                             qrow0, nch,
                                    smem + L.mrg, red, misc + 1, DH);

  // ---- 6. the append (subgroup 0; no workgroup reads that slot in this
  // launch).  Last, because nothing may wait for these stores: vmcnt counts
  // stores too, and a wait placed after them for an older load would hold
  // the fold and the merge until the stores complete. ----
  if (is_new && sub == 0 && (Q8 ? w == 0 : tid < DH)) {  // (d = 512: tid, tid + NT)
    const int slot_row = n - 1;
    int64_t off, soff;  // element (Q8: byte) offset of the row; Q8: of its scale
    if constexpr (PAGED) {
      const int64_t blk = a.block_table[(int64_t)b * a.max_blocks + (slot_row >> a.page_shift)];
      const int sl = slot_row & ((1 << a.page_shift) - 1);
      off = blk * a.block_stride + hoff + (int64_t)sl * a.tok_stride;
      soff = blk * a.block_stride + a.sc_off + h * a.sc_head + 4 * sl;
    } else {
      off = (int64_t)slot_row * a.tok_stride + hoff;
      soff = (int64_t)slot_row * a.tok_stride + a.sc_off + h * a.sc_head;
    }
    if constexpr (Q8) {
#pragma unroll
      for (int e = 0; e < D / 64; ++e) {
        if (lane + 64 * e >= DH) continue;  // a padded row ends at DH codes
        reinterpret_cast<int8_t*>(a.k)[off + lane + 64 * e] = (int8_t)kcode[e];
        reinterpret_cast<int8_t*>(a.v)[off + lane + 64 * e] = (int8_t)vcode[e];
      }
      if (lane == 0) {
        *reinterpret_cast<float*>(reinterpret_cast<char*>(a.k) + soff) = kscale;
        *reinterpret_cast<float*>(reinterpret_cast<char*>(a.v) + soff) = vscale;
      }
    } else if constexpr (sizeof(T) == 2) {  // exact bf16 values: the rounding returns their bits
      for (int j = tid; j < DH; j += NT) {
        reinterpret_cast<uint16_t*>(a.k)[off + j] = f32_to_bf16(knew[j]);
        reinterpret_cast<uint16_t*>(a.v)[off + j] = f32_to_bf16(vnew[j]);
      }
    } else {
      for (int j = tid; j < DH; j += NT) {
        reinterpret_cast<float*>(a.k)[off + j] = knew[j];
        reinterpret_cast<float*>(a.v)[off + j] = vnew[j];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// bf16 KV on the matrix cores.
//
// A wave takes tiles of 32 cache rows of the workgroup's KV head (claimed
// like the blocks of attn_kernel) and keeps the GH <= 16 query heads of the
// group on the 16 columns of v_mfma_f32_16x16x32_bf16:
//   scores  S^T (32 rows x 16 heads) = K (32 x D) . Q^T (D x 16), two 16-row
//           halves, D/32 k-steps each.  K goes from HBM straight into the A
//           operand: lane l holds row l%16 and elements 8*(l/16)..+7 of a
//           32-wide k-step, one 16-byte load.  q (fp32) enters as three bf16
//           pieces hi + mid + lo, which together hold its 24-bit significand,
//           so the scores are the fp32 products of q with the bf16 K summed
//           in fp32.
//   softmax the accumulator of a half holds, in lane l, head l%16 and rows
//           4*(l/16)+r: a lane owns one head and 8 rows of the tile, and the
//           online max / rescale run in place (max across the 4 lanes of a
//           head by two shuffles).
//   PV      O^T (D x 16) += V^T (D x 32) . P^T (32 x 16) per 16-row block of
//           O^T.  The k index of this product runs over the tile's rows in
//           the order tau(g, e) = 16*(e/4) + 4g + e%4 (g = l/16): exactly the
//           8 probabilities lane l already holds, so P is the B operand as it
//           stands (again as bf16 hi + mid + lo).  V is staged in LDS
//           (row-major, 16-byte units XOR-swizzled by row: vt_off) and read
//           back with ds_read_b64_tr_b16: lane l reads 8 bytes of row l/4
//           (+16) at column 16*dt + 4*(l%4), and the transpose hands lane i of
//           each 16-lane group element i%4 of lane 4e+i/4's read as slot e,
//           i.e. V[tau(g, e)][16*dt + i]: the A operand.
// Prologue, new token and chunk output are those of attn_kernel.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));

constexpr int kMfmaWaves = 4;                  // waves per workgroup
constexpr int kMfmaThreads = kMfmaWaves * 64;
constexpr int kTile = 32;                      // cache rows per wave step

template <int D>
constexpr int kMfmaQStride = D + 4;

// LDS of attn_mfma_kernel, in floats.  vt: per wave, 32 staged V rows of D
// bf16 (16*D floats), which after the stream hold the wave's partial o;
// sc (Q8): per wave, the K then the V row scales of its current tile.
struct LdsM {
  int qs, cs, sn, knew, vnew, nw, wm, wl, sc, vt, blk, misc, mrg, total;
  __host__ __device__ LdsM(int D, int GH, int chunk, int page_shift, bool paged, bool q8,
                           int merge) {
    int o = 0;
    qs = o; o += GH * (D + 4);  // rows kMfmaQStride<D> = D + 4 floats apart
    cs = o; o += D / 2;
    sn = o; o += D / 2;
    knew = o; o += D;
    vnew = o; o += D;
    nw = o; o += D;  // k norm weights
    wm = o; o += kMfmaWaves * GH;
    wl = o; o += kMfmaWaves * GH;
    o = (o + 3) & ~3;
    sc = o; o += q8 ? kMfmaWaves * 2 * kTile : 0;
    o = (o + 63) & ~63;  // 256-byte aligned: the swizzle's bank pattern
    vt = o; o += kMfmaWaves * kTile * D / 2;
    blk = o; o += paged ? ((chunk >> page_shift) + 2) : 0;
    misc = o; o += 8;  // tile claim counter, merge flag
    mrg = o; o += merge;  // in-launch merge: chunk statistics
    total = o;
  }
};

// Byte offset of 16-byte unit ch (elements 8ch .. 8ch+7) of staged V row r:
// unit ch of the row is stored at unit ch ^ f(r).  Measured on MI355X
// (SQ_LDS_BANK_CONFLICT of each access pattern alone), a 16-byte LDS store
// serves 8 lanes a cycle and conflicts unless their addresses fall in
// distinct 16-byte slots mod 128 bytes, and ds_read_b64_tr_b16 serves 32
// lanes a cycle, distinct 8-byte slots mod 256 bytes.  The stores put rows
// r0 .. r0+7 of one unit ch in 8 lanes: distinct when the low 3 bits of f
// run over 8 values; a transposed read takes units 2dt and 2dt+1 of 8 rows:
// 16 distinct units of a 256-byte span when f >> 1 runs over 8 values.
// D = 128 or 256 (16 or 32 units a row): f(r) = 2(r%8) + (r/4)%2 meets
// both; D = 64 (8 units, 2 rows per 256 bytes): f(r) = r%8.  The
// 32-byte-segment swizzle this replaces conflicted 2-way on every store.
template <int D>
__device__ __forceinline__ int vt_f(int r) {
  return D != 64 ? (((r & 7) << 1) | ((r >> 2) & 1)) : (r & 7);
}
template <int D>
__device__ __forceinline__ int vt_off(int r, int ch) {
  return r * (2 * D) + 16 * (ch ^ vt_f<D>(r));
}

// Byte offset of 16-byte unit ch of a staged K row (the prefill's A operand
// of the scores, read by 16-byte loads of 16 keys at one unit): unit ch of
// key r at ch ^ (r % 16) (D = 64: r % 8).  Measured, a 16-byte LDS read
// serves 16 lanes a cycle, conflict-free on 16 distinct units mod 256 bytes.
template <int D>
__device__ __forceinline__ int kt_f(int r) {
  return D == 64 ? (r & 7) : (r & 15);
}
template <int D>
__device__ __forceinline__ int kt_off(int r, int ch) {
  return r * (2 * D) + 16 * (ch ^ kt_f<D>(r));
}

// x = hi + mid + lo in bf16 (round to nearest even at each step); the three
// pieces carry the full fp32 significand.
__device__ __forceinline__ void split3(float x, __bf16& hi, __bf16& mid, __bf16& lo) {
  hi = (__bf16)x;
  float r = x - (float)hi;
  mid = (__bf16)r;
  r -= (float)mid;
  lo = (__bf16)r;
}

__device__ __forceinline__ f32x4 mfma_bf16(bf16x8_t a, bf16x8_t b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4 mfma_f16(f16x8_t a, f16x8_t b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 16 int8 codes -> 16 bf16 (exact: |code| <= 127), bytes 0-7 into lo, 8-15
// into hi, each in memory order.  One v_cvt_pk_bf16_f32 per pair (its
// rounding is the identity on these values).
__device__ __forceinline__ void i8x16_to_bf16(const u32x4& x, u32x4& lo, u32x4& hi) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w = x[i];
    const float f0 = (float)(int8_t)(w & 0xFF), f1 = (float)(int8_t)((w >> 8) & 0xFF);
    const float f2 = (float)(int8_t)((w >> 16) & 0xFF), f3 = (float)((int32_t)w >> 24);
    u32x4& dst = i < 2 ? lo : hi;
    dst[2 * (i & 1)] = bf16_pair_exact(f0, f1);
    dst[2 * (i & 1) + 1] = bf16_pair_exact(f2, f3);
  }
}

// Matrix-core decode over a bf16 (Q8 = false) or Q8 (Q8 = true) cache.
//
// Q8: each lane reads 16 codes per 16-byte load, covering two k-steps: load
// j of lane group g holds row bytes 64j + 16g .. +15, so k-step kk, element
// e is head-dim index 64*(kk/2) + 16g + 8*(kk%2) + e, and q^T takes the same
// order.  Codes widen to bf16 exactly; a score is (codes . q) * s_k * scale,
// and the PV operand is p * s_v in the same three bf16 pieces as bf16's p
// (the row sum l takes p itself).  Lane (row l%16) loads its A-row's two
// scales; they pass through a per-wave LDS slot to the accumulator lanes of
// rows 16u + 4*(l/16) + r.  The new token's k (rotated) and v rows are
// quantized in the workgroup like the cache rows and folded in as code * s.
template <int D, int GH, bool PAGED, bool ROPE, bool Q8>
__global__ __launch_bounds__(kMfmaThreads, 2) void attn_mfma_kernel(AttnArgs a) {
  static_assert(D == 64 || D == 128, "MFMA tiles cover D = 64 or 128");
  static_assert(GH >= 1 && GH <= 16, "the group's q heads on the 16 MFMA columns");
  constexpr int NW = kMfmaWaves, NT = kMfmaThreads;
  constexpr int KK = D / 32;  // k-steps of the score product
  constexpr int DT = D / 16;  // 16-row blocks of O^T
  constexpr int RS = kTile * D / 2;  // floats of a wave's LDS region
  constexpr int KL = Q8 ? D / 64 : KK;  // 16-byte loads per row and lane (K or V)
  using E = typename std::conditional<Q8, int8_t, bf16_t>::type;

  constexpr int DH = D;  // never padded
  constexpr int QSTR = kMfmaQStride<D>;  // floats between q rows in LDS
  extern __shared__ float smem[];
  const LdsM L(D, GH, a.chunk, a.page_shift, PAGED, Q8, a.mrg);
  float* qs = smem + L.qs;
  float* knew = smem + L.knew;
  float* vnew = smem + L.vnew;
  int* misc = reinterpret_cast<int*>(smem + L.misc);

  // chunk slot z (chunk c = nch - 1 - z, below), (KV head, subgroup) index
  // hs and sequence b of this workgroup
  const int G = a.nq / a.nkv;
  const int nsub = G / GH;
  int z, hs, b;
  if (a.chunk_fast) {  // workgroup id runs on XCD id % 8 (launch_pair)
    const int HS = a.nkv * nsub;
    const int k = (int)(blockIdx.x >> 3);
    // (sequence, chunk) pair pi = (k / HS) * 8 + id % 8, chunk slot slowest;
    // padded ids (z >= nchunks) exit below
    const int pi = (k / HS) * 8 + (int)(blockIdx.x & 7);
    z = pi / a.nseq;
    b = pi - z * a.nseq;
    hs = k % HS;
  } else if (a.xmap) {  // slot id % 8 runs on XCD id % 8 (launch_pair); padding ids exit
    const int s8 = (int)(blockIdx.x & 7);
    if (s8 >= a.slots) return;
    z = (int)(blockIdx.x >> 3);
    hs = s8 % (a.nkv * nsub);
    b = s8 / (a.nkv * nsub);
  } else {
    z = blockIdx.z;
    hs = blockIdx.x;
    b = blockIdx.y;
  }
  const int sub = hs % nsub;
  const int h = hs / nsub;
  const int hq0 = h * G + sub * GH;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int m16 = lane & 15, g4 = lane >> 4;

  int n = a.n, t0 = a.t0, pos = a.pos;
  if constexpr (PAGED) {
    n = a.seq_lens[b];
    pos = a.pos_arr ? a.pos_arr[b] : n - 1;
    t0 = (a.window > 0 && pos - a.window + 1 > 0) ? pos - a.window + 1 : 0;
    if (t0 > n) t0 = n;
  }
  const bool fold = ROPE && a.fold;  // this launch appends and folds in the new token
  const int cend = fold ? n - 1 : n;
  int nch = a.nchunks;
  if constexpr (PAGED) {
    const int span = cend - t0;
    nch = span > 0 ? (span + a.chunk - 1) / a.chunk : (fold ? 1 : 0);
    if (nch > a.nchunks) nch = a.nchunks;
  }
  if (z >= nch) {
    if (z == 0) {  // empty attended range: o = 0, and q normed and rotated (empty_range_q)
      for (int i = tid; i < GH * D; i += NT) a.o[((int64_t)b * a.nq + hq0) * D + i] = 0.f;
      if (ROPE && !fold && a.q_out) empty_range_q<NT>(a, (int64_t)b * a.nq + hq0, GH, D, pos, smem);
    }
    return;
  }
  const int c = nch - 1 - z;  // the new token's chunk first, as in attn_kernel
  const int tb = t0 + c * a.chunk;
  const int cntg = max(0, min(a.chunk, cend - tb));
  const bool is_new = fold && c == nch - 1;
  const bool split = nch > 1;
  const int64_t slot = (int64_t)b * a.nkv * nsub + hs;

  const E* __restrict__ Kb = reinterpret_cast<const E*>(a.k);
  const E* __restrict__ Vb = reinterpret_cast<const E*>(a.v);
  const int64_t hoff = (int64_t)h * a.head_stride;
  const int64_t qrow0 = (int64_t)b * a.nq + hq0;

  // ---- prologue ----
  if constexpr (PAGED) {
    int32_t* sblk_w = reinterpret_cast<int32_t*>(smem + L.blk);
    const int p0 = tb >> a.page_shift;
    const int p1 = max(p0, (tb + cntg - 1) >> a.page_shift);
    for (int i = tid; i <= p1 - p0; i += NT)
      sblk_w[i] = a.block_table[(int64_t)b * a.max_blocks + p0 + i];
    lds_barrier();
  }
  const int32_t* sblk = reinterpret_cast<const int32_t*>(smem + L.blk);
  auto row_ptr = [&](const E* base, int t) -> const E* {
    if constexpr (PAGED) {
      const int pg = (t >> a.page_shift) - (tb >> a.page_shift);
      return base + (int64_t)sblk[pg] * a.block_stride + hoff +
             (int64_t)(t & ((1 << a.page_shift) - 1)) * a.tok_stride;
    } else {
      return base + (int64_t)t * a.tok_stride + hoff;
    }
  };
  // Q8: the fp32 scale of row t of head h
  auto sc_ptr = [&](const E* base, int t) -> const float* {
    const char* p = reinterpret_cast<const char*>(base) + a.sc_off + h * a.sc_head;
    if constexpr (PAGED) {
      const int pg = (t >> a.page_shift) - (tb >> a.page_shift);
      return reinterpret_cast<const float*>(p + (int64_t)sblk[pg] * a.block_stride) +
             (t & ((1 << a.page_shift) - 1));
    } else {
      return reinterpret_cast<const float*>(p + (int64_t)t * a.tok_stride);
    }
  };
  // Row mapping.  Paged: the chunk's rows [tb, tb + cntg), in order.  A
  // contiguous cache: tile k of chunk c is the range's 32-row tile
  // c + k*nch (cyclic), so at any moment the launch's workgroups read
  // neighbouring tiles (a streaming probe of c5's layout: 5.17 TB/s with
  // each chunk one block of rows, 5.78 TB/s cyclic).  Rows past the end load
  // the last row of the range (the first of an empty one): every wave issues
  // the same loads on every path.
  const int rlim = PAGED ? cntg : cend - t0;  // rows of the chunk / of the whole range
  const int rfirst = PAGED ? tb : t0;
  const int rmax = max(rlim - 1, 0);
  int ntiles;
  if constexpr (PAGED) {
    ntiles = (cntg + kTile - 1) / kTile;
  } else {
    const int gt = (rlim + kTile - 1) / kTile;  // tiles of the range
    ntiles = c < gt ? (gt - 1 - c) / nch + 1 : 0;
  }
  auto tile_row = [&](int tile) -> int {  // first row of a tile, from rfirst
    return PAGED ? tile * kTile : (c + tile * nch) * kTile;
  };
  u32x4 kr[2][KL], vr[2][KL];
  float skr[2] = {0.f, 0.f}, svr[2] = {0.f, 0.f};  // Q8: scales of this lane's A-rows
  // Rows load without the streaming hint here (measured: c4 bf16 -8%, c5q8
  // -16% kernel time): Q8 KV heads share lines (the token's scales; in a
  // token-major cache, the head rows too), so a line fetched for one head
  // has to stay in L2 for the next, and the paged rows gain as well.
  auto load_tile = [&](int tile) {
    if constexpr (Q8) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int t = rfirst + min(tile_row(tile) + 16 * u + m16, rmax);
        skr[u] = *sc_ptr(Kb, t);
        svr[u] = *sc_ptr(Vb, t);
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = rfirst + min(tile_row(tile) + 16 * u + m16, rmax);
      const E* pk = row_ptr(Kb, t);
      const E* pv = row_ptr(Vb, t);
      if constexpr (Q8) {
#pragma unroll
        for (int j = 0; j < KL; ++j)
          kr[u][j] = *reinterpret_cast<const u32x4*>(pk + 64 * j + 16 * g4);
#pragma unroll
        for (int j = 0; j < KL; ++j)
          vr[u][j] = *reinterpret_cast<const u32x4*>(pv + 16 * (g4 + 4 * j));
      } else {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
          kr[u][kk] = *reinterpret_cast<const u32x4*>(pk + 32 * kk + 8 * g4);
#pragma unroll
        for (int q = 0; q < KK; ++q)
          vr[u][q] = *reinterpret_cast<const u32x4*>(pv + 8 * (g4 + 4 * q));
      }
    }
  };
  constexpr int QV = GH * D / 4;
  constexpr int QPT = (QV + NT - 1) / NT;
  static_assert(D <= NT, "one thread per head-dim element in the prologue");
  f32x4 qv[QPT];
#pragma unroll
  for (int u = 0; u < QPT; ++u)
    qv[u] = reinterpret_cast<const f32x4*>(a.q + qrow0 * D)[min(tid + u * NT, QV - 1)];
  float invf = 0.f, knv = 0.f, vnv = 0.f, kwv = 0.f;
  f32x4 qwt[QPT];  // q norm weights of this thread's q elements
  if constexpr (ROPE) {
    // every path issues these loads: a layer without RoPE (inv_freq NULL)
    // or without an append reads q in their place (nq >= nkv rows), unused
    const float* ivp = a.inv_freq ? a.inv_freq : a.q;
    const float* knp = fold ? a.k_new : a.q;
    const float* vnp = fold ? a.v_new : a.q;
    invf = ivp[min(tid, D / 2 - 1)];
    knv = knp[((int64_t)b * a.nkv + h) * D + min(tid, D - 1)];
    vnv = vnp[((int64_t)b * a.nkv + h) * D + min(tid, D - 1)];
    if (a.q_norm) {
#pragma unroll
      for (int u = 0; u < QPT; ++u)
        qwt[u] = reinterpret_cast<const f32x4*>(a.q_norm)[min(tid + u * NT, QV - 1) % (D / 4)];
    }
    if (is_new && a.k_norm) kwv = a.k_norm[min(tid, D - 1)];
  }
  float vq[kVnPT];
  const bool vn = ROPE && is_new && a.v_norm;  // uniform over the workgroup
  if (vn) v_norm_load<D, NT>(a, b, tid, vq, DH);
  int tile = w;  // each wave's first tile; the rest are claimed
  load_tile(tile);
  if (tid == 0) misc[0] = NW;
  if constexpr (ROPE) {
    if (a.q_norm) q_norm_regs<D, QPT>(a, qv, qwt, DH);
  }
#pragma unroll
  for (int u = 0; u < QPT; ++u) {
    const int i = tid + u * NT;
    if (i < QV) *reinterpret_cast<f32x4*>(qs + (i / (D / 4)) * QSTR + 4 * (i % (D / 4))) = qv[u];
  }
  if constexpr (ROPE) {
    float* csn = smem + L.cs;
    float* sn = smem + L.sn;
    const bool rot = a.inv_freq != nullptr;  // uniform: no RoPE on a NoPE layer
    if (rot && tid < D / 2) {
      const float ang = (float)pos * invf;
      double sd, cd;
      sincos((double)ang, &sd, &cd);
      csn[tid] = (float)cd;
      sn[tid] = (float)sd;
    }
    if (is_new && tid < D) {
      knew[tid] = knv;
      vnew[tid] = vnv;
    }
    if (vn) v_norm_share<D, NT>(a, b, tid, w, lane, vq, smem + L.wl, DH);
    if (tid < D) smem[L.nw + tid] = kwv;
    if (is_new && a.k_norm) k_norm_share(w, lane, tid < D ? knv * knv : 0.f, smem + L.wm);
    lds_barrier();
    for (int i = tid; rot && i < GH * (D / 2); i += NT) {
      const int g = i / (D / 2), j = i - g * (D / 2);
      const float x0 = qs[g * QSTR + j], x1 = qs[g * QSTR + j + D / 2];
      qs[g * QSTR + j] = x0 * csn[j] - x1 * sn[j];
      qs[g * QSTR + j + D / 2] = x0 * sn[j] + x1 * csn[j];
    }
    if (is_new) {
      const NewNorms nn = new_norms<D, NW>(a, smem + L.wm, smem + L.wl, DH);
      for (int j = tid; j < D / 2; j += NT) {
        float k0 = knew[j], k1 = knew[j + D / 2];
        float v0 = vnew[j], v1 = vnew[j + D / 2];
        nn.apply(a, smem + L.nw, j, D / 2, k0, k1, v0, v1);
        const float r0 = rot ? k0 * csn[j] - k1 * sn[j] : k0;
        const float r1 = rot ? k0 * sn[j] + k1 * csn[j] : k1;
        if constexpr (Q8) {  // quantized after the stream (whole rows)
          knew[j] = r0;
          knew[j + D / 2] = r1;
          vnew[j] = v0;
          vnew[j + D / 2] = v1;
        } else {
          knew[j] = __uint_as_float((uint32_t)f32_to_bf16(r0) << 16);
          knew[j + D / 2] = __uint_as_float((uint32_t)f32_to_bf16(r1) << 16);
          vnew[j] = __uint_as_float((uint32_t)f32_to_bf16(v0) << 16);
          vnew[j + D / 2] = __uint_as_float((uint32_t)f32_to_bf16(v1) << 16);
        }
      }
    }
  }
  lds_barrier();

  int next_fixed = w + NW;
  auto claim = [&]() -> int {
    if (!a.dynamic) {
      const int v = next_fixed;
      next_fixed += NW;
      return v;
    }
    int v = 0;
    if (lane == 0) v = atomicAdd(&misc[0], 1);
    return __builtin_amdgcn_readfirstlane(v);
  };

  // q^T as the B operand: lane l holds head l%16 (zero past GH), elements
  // 32*kk + 8*(l/16) + e (Q8: 64*(kk/2) + 16*(l/16) + 8*(kk%2) + e), scaled
  // by scale*log2(e), in three bf16 pieces.  16-byte reads of rows QSTR =
  // D + 4 floats apart: the 8 lanes of a read (heads r .. r+7) fall in 8
  // distinct 16-byte slots (rows of D floats: one slot, 8-way conflicts).
  const float qsc = a.scale * kLog2e;
  bf16x8_t qh[KK], qm[KK], ql[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk)
#pragma unroll
    for (int e4 = 0; e4 < 8; e4 += 4) {
      const int di = Q8 ? 64 * (kk >> 1) + 16 * g4 + 8 * (kk & 1) + e4 : 32 * kk + 8 * g4 + e4;
      const f32x4 x4 = m16 < GH ? *reinterpret_cast<const f32x4*>(qs + m16 * QSTR + di)
                                : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        __bf16 hi, mid, lo;
        split3(x4[e] * qsc, hi, mid, lo);
        qh[kk][e4 + e] = hi;
        qm[kk][e4 + e] = mid;
        ql[kk][e4 + e] = lo;
      }
    }

  // ---- stream ----
  char* vt = reinterpret_cast<char*>(smem + L.vt + w * RS);
  f32x4 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  float* scw = smem + L.sc + w * (2 * kTile);  // Q8: this wave's scale slots
  while (tile < ntiles) {
    // V rows into this wave's LDS region (lane: row 16u + l%16, 16-byte
    // units l/16 + 4q), swizzled by vt_off
    f32x4 sk4[2], sv4[2];  // Q8: scales of accumulator rows 16u + 4*(l/16) + r
    if constexpr (Q8) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int j = 0; j < KL; ++j) {
          // load j holds row bytes 16*(l/16 + 4j): 32-byte bf16 segment l/16 + 4j
          const int r = 16 * u + m16, s = g4 + 4 * j;
          u32x4 lo, hi;
          i8x16_to_bf16(vr[u][j], lo, hi);
          *reinterpret_cast<u32x4*>(vt + vt_off<D>(r, 2 * s)) = lo;
          *reinterpret_cast<u32x4*>(vt + vt_off<D>(r, 2 * s + 1)) = hi;
        }
      if (g4 == 0) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          scw[16 * u + m16] = skr[u];
          scw[kTile + 16 * u + m16] = svr[u];
        }
      }
      // the slots are this wave's own: LDS keeps its order, and the fence
      // keeps the compiler from moving the reads above the writes
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        sk4[u] = *reinterpret_cast<const f32x4*>(scw + 16 * u + 4 * g4);
        sv4[u] = *reinterpret_cast<const f32x4*>(scw + kTile + 16 * u + 4 * g4);
      }
    } else {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int q = 0; q < KK; ++q) {
          const int r = 16 * u + m16, ch = g4 + 4 * q;
          *reinterpret_cast<u32x4*>(vt + vt_off<D>(r, ch)) = vr[u][q];
        }
    }
    // scores of the two 16-row halves
    f32x4 sacc[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      sacc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
      if constexpr (Q8) {
#pragma unroll
        for (int j = 0; j < KL; ++j) {
          u32x4 lo, hi;
          i8x16_to_bf16(kr[u][j], lo, hi);
          const bf16x8_t k0 = __builtin_bit_cast(bf16x8_t, lo);
          const bf16x8_t k1 = __builtin_bit_cast(bf16x8_t, hi);
          sacc[u] = mfma_bf16(k0, ql[2 * j], sacc[u]);
          sacc[u] = mfma_bf16(k0, qm[2 * j], sacc[u]);
          sacc[u] = mfma_bf16(k0, qh[2 * j], sacc[u]);
          sacc[u] = mfma_bf16(k1, ql[2 * j + 1], sacc[u]);
          sacc[u] = mfma_bf16(k1, qm[2 * j + 1], sacc[u]);
          sacc[u] = mfma_bf16(k1, qh[2 * j + 1], sacc[u]);
        }
      } else {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          const bf16x8_t kv = __builtin_bit_cast(bf16x8_t, kr[u][kk]);
          sacc[u] = mfma_bf16(kv, ql[kk], sacc[u]);
          sacc[u] = mfma_bf16(kv, qm[kk], sacc[u]);
          sacc[u] = mfma_bf16(kv, qh[kk], sacc[u]);
        }
      }
    }
    // the next tile's loads go out while this one is finished
    const int nx = claim();
    if (nx < ntiles) load_tile(nx);
    // online softmax (base 2) on the accumulators: lane = head l%16, rows
    // 16u + 4*(l/16) + r
    float sv[2][4];
    float tmax = -INFINITY;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = tile_row(tile) + 16 * u + 4 * g4 + r;
        sv[u][r] = row < rlim ? (Q8 ? sacc[u][r] * sk4[u][r] : sacc[u][r]) : -INFINITY;
        tmax = fmaxf(tmax, sv[u][r]);
      }
    tmax = max_xor32(max_xor16(tmax));
    // finite: a claimed tile has a row; the first tile always moves the max
    if (__builtin_amdgcn_ballot_w64(tmax > m_run + kLazyMax) != 0) {
      const float mn = fmaxf(m_run, tmax);
      const float alpha = exp2_hw(m_run - mn);
      m_run = mn;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
    }
    bf16x8_t ph, pm, pl;
    float ps = 0.f;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = exp2_hw(sv[u][r] - m_run);
        ps += p;
        __bf16 hi, mid, lo;
        split3(Q8 ? p * sv4[u][r] : p, hi, mid, lo);
        ph[4 * u + r] = hi;
        pm[4 * u + r] = mid;
        pl[4 * u + r] = lo;
      }
    l_run += ps;
    __builtin_amdgcn_wave_barrier();
    // PV: V^T of the 16-row block dt by two transposed reads
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      i16x4_t t2[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int r = (lane >> 2) + 16 * u;
        t2[u] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4_t*)(
                vt + vt_off<D>(r, 2 * dt + ((lane & 3) >> 1)) + 8 * (lane & 1)));
      }
      const bf16x8_t av = __builtin_bit_cast(
          bf16x8_t, __builtin_shufflevector(t2[0], t2[1], 0, 1, 2, 3, 4, 5, 6, 7));
      o[dt] = mfma_bf16(av, pl, o[dt]);
      o[dt] = mfma_bf16(av, pm, o[dt]);
      o[dt] = mfma_bf16(av, ph, o[dt]);
    }
    __builtin_amdgcn_wave_barrier();
    tile = nx;
  }

  // ---- the new token: folded in by wave 0 (appended by subgroup 0 at the
  // very end, like attn_kernel's append: nothing may wait for those stores) ----
  [[maybe_unused]] int kcode[D / 64], vcode[D / 64];  // Q8: the row's codes
  [[maybe_unused]] float kscale = 0.f, vscale = 0.f;  // Q8: and scales
  if constexpr (Q8) {
    if (is_new && w == 0) {
      // quantize the k and v rows as the cache holds them; LDS gets code * s
      constexpr int EPL = D / 64;
      float kx[EPL], vx[EPL];
      float ka = 0.f, va = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        kx[e] = knew[lane + 64 * e];
        vx[e] = vnew[lane + 64 * e];
        ka = fmaxf(ka, fabsf(kx[e]));
        va = fmaxf(va, fabsf(vx[e]));
      }
      kscale = q8_scale(group_max<64>(ka));
      vscale = q8_scale(group_max<64>(va));
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        kcode[e] = q8_code(kx[e], kscale);
        vcode[e] = q8_code(vx[e], vscale);
        knew[lane + 64 * e] = (float)kcode[e] * kscale;
        vnew[lane + 64 * e] = (float)vcode[e] * vscale;
      }
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");  // the fold reads other lanes' rows
    }
  }
  if (is_new && w == 0) {
    float part = 0.f;
    if (m16 < GH) {
#pragma unroll 8
      for (int d = g4 * (D / 4); d < (g4 + 1) * (D / 4); ++d)
        part = fmaf(qs[m16 * QSTR + d], knew[d], part);
    }
    part = sum_xor32(sum_xor16(part));
    const float snew = part * qsc;  // base 2, as the streamed scores
    const float mn = fmaxf(m_run, snew);
    const float alpha = exp2_hw(m_run - mn);
    const float p = exp2_hw(snew - mn);
    m_run = mn;
    l_run = l_run * alpha + (g4 == 0 ? p : 0.f);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) o[dt][r] = o[dt][r] * alpha + p * vnew[16 * dt + 4 * g4 + r];
  }

  // ---- the wave's partial into its own LDS region, then the chunk ----
  l_run = sum_xor32(sum_xor16(l_run));
  float* wm = smem + L.wm;
  float* wl = smem + L.wl;
  float* red = smem + L.vt;
  if (m16 < GH) {
    if (g4 == 0) {
      wm[w * GH + m16] = m_run * kLn2;  // natural units for the merge
      wl[w * GH + m16] = l_run;
    }
    // head m16's row with its float index XOR 4*(m16 % 8): the 8 lanes of a
    // store then hit distinct 16-byte slots (rows of D floats alone: 8-way)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      *reinterpret_cast<f32x4*>(red + w * RS + m16 * D + ((16 * dt + 4 * g4) ^ (4 * (m16 & 7)))) =
          o[dt];
  }
  lds_barrier();
  finish_chunk<D, GH, NW, NT, ROPE, NW * RS, true, QSTR>(a, wm, wl, red, RS, qs, tid, lane, split, slot, c,
                                              qrow0, nch,
                                    smem + L.mrg, red, misc + 1, DH);

  // ---- the append, last ----
  const bool store_new = is_new && sub == 0 && (Q8 ? w == 0 : tid < D);
  if (store_new) {
    const int slot_row = n - 1;
    int64_t off, soff;  // element (Q8: byte) offset of the row; Q8: of its scale
    if constexpr (PAGED) {
      const int64_t blk = a.block_table[(int64_t)b * a.max_blocks + (slot_row >> a.page_shift)];
      const int sl = slot_row & ((1 << a.page_shift) - 1);
      off = blk * a.block_stride + hoff + (int64_t)sl * a.tok_stride;
      soff = blk * a.block_stride + a.sc_off + h * a.sc_head + 4 * sl;
    } else {
      off = (int64_t)slot_row * a.tok_stride + hoff;
      soff = (int64_t)slot_row * a.tok_stride + a.sc_off + h * a.sc_head;
    }
    if constexpr (!Q8) {
      reinterpret_cast<uint16_t*>(a.k)[off + tid] = f32_to_bf16(knew[tid]);
      reinterpret_cast<uint16_t*>(a.v)[off + tid] = f32_to_bf16(vnew[tid]);
    } else {
#pragma unroll
      for (int e = 0; e < D / 64; ++e) {
        reinterpret_cast<int8_t*>(a.k)[off + lane + 64 * e] = (int8_t)kcode[e];
        reinterpret_cast<int8_t*>(a.v)[off + lane + 64 * e] = (int8_t)vcode[e];
      }
      if (lane == 0) {
        *reinterpret_cast<float*>(reinterpret_cast<char*>(a.k) + soff) = kscale;
        *reinterpret_cast<float*>(reinterpret_cast<char*>(a.v) + soff) = vscale;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Causal prefill attention (include/molot/gemm.h:409-446) on the matrix cores.
//
// The query rows of one KV head are r = m*G + g: token m (position pos0 + m)
// and q head h*G + g of the group.  A workgroup of 4 waves owns 64
// consecutive rows, wave w the 16 rows w*16.. on the 16 columns of the
// matrix instructions.  It streams the keys its rows attend, 32 per tile,
// through LDS, with the next tile's global loads in flight while the
// current one is used; each row is masked to its own causal end
// min(pos+1, N) and window start.  Query blocks run from the last (most
// keys) to the first, heads fastest across the grid.
// The reference's exps are libm expf summed in double with the weights
// normalised before PV; here the hardware base-2 exp of scores pre-scaled by
// log2(e), fp32 running sums with a lazy max rescale, and one division at
// the end (fp32 rounding differences).
struct PfArgs {
  const float* q;  // [M][nq][D]
  const void* k;   // token-major cache [N][nkv*D], or pages [block][nkv][page][D]
  const void* v;
  float* o;        // [M][nq][D]
  const int32_t* block_table;  // paged: the sequence's row of block ids
  int nq, nkv, M, N, pos0, window, nqb;  // nqb: blocks of 16 * (waves) query rows per KV head
  int dh;  // head dim as stored (< D: the launch runs padded to D, through the pieces)
  int page_shift;
  float scale;
  // the attended keys [T0, T0 + R) of every KV head split into 16-bit pieces
  // once for the launch (pf_split_kernel): [K, V][nkv][3 pieces][R][D]; NULL:
  // the kernel splits each staged tile itself
  const uint16_t* pieces;
  int T0, R;
  int Rsplit;  // pf_split_kernel splits rows [T0, T0 + Rsplit); the appending step wrote the rest
  // split-K over the key tiles (nsplit > 1): split s of a query block takes
  // its share of the tiles and writes unnormalised o and (max, sum) per query
  // row, slot m*nq + head, to part_o [slot][nsplit][D] and part_ml
  // [slot][nsplit][2]; combine_kernel merges them into O
  int nsplit;
  float* part_o;
  float* part_ml;
};

// Cache offset (elements of T; Q8: bytes) of row t of KV head h, and for Q8
// the byte offset of its scale (soff).  Token-major: [N][nkv*D] (Q8 rows of
// nkv*D codes, then nkv scales padded to 16 bytes); paged: blocks of
// [nkv][page][D] (Q8: [nkv][page][D] codes, then [nkv][page] scales).
template <int D, typename T, bool PAGED>
__device__ __forceinline__ int64_t pf_row_off(const PfArgs& a, int h, int t, int64_t& soff) {
  constexpr bool Q8 = std::is_same<T, q8_t>::value;
  const int pg = 1 << a.page_shift;
  const int64_t R = (int64_t)a.nkv * D + ((4 * a.nkv + 15) & ~15);
  const int64_t BB = (int64_t)a.nkv * pg * (D + 4);
  if constexpr (PAGED) {
    const int64_t blk = a.block_table[t >> a.page_shift];
    const int sl = t & (pg - 1);
    if constexpr (Q8) {
      soff = blk * BB + (int64_t)a.nkv * pg * D + 4 * ((int64_t)h * pg + sl);
      return blk * BB + ((int64_t)h * pg + sl) * D;
    }
    return ((blk * a.nkv + h) * pg + sl) * (int64_t)a.dh;
  } else {
    if constexpr (Q8) {
      soff = (int64_t)t * R + (int64_t)a.nkv * D + 4 * h;
      return (int64_t)t * R + (int64_t)h * D;
    }
    return ((int64_t)t * a.nkv + h) * (int64_t)a.dh;
  }
}

// K and V of the keys [T0, T0 + R) as pieces (the values the prefill kernel
// would split per tile: fp32 rows, or Q8 code * s), into [K, V][nkv][3][R][D]
// (16-bit elements): K and V rows as two fp16 pieces of the row scaled by a
// power of two (split2h), the rows' units (floats) side by side at the start
// of the third.  Thread: one 8-element unit of one row, a row's D/8 units in
// consecutive lanes; grid (units / 256, nkv, 2).
template <int D, typename T, bool PAGED>
__global__ __launch_bounds__(256) void pf_split_kernel(PfArgs a, uint16_t* out) {
  constexpr bool Q8 = std::is_same<T, q8_t>::value;
  static_assert(sizeof(T) != 2, "bf16 caches are exact in one piece");
  constexpr int UPR = D / 8;
  const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (u >= (int64_t)a.Rsplit * UPR) return;
  const int h = blockIdx.y, kv = blockIdx.z;
  const int r = (int)(u / UPR), j = (int)(u - (int64_t)r * UPR);
  int64_t soff = 0;
  const int64_t off = pf_row_off<D, T, PAGED>(a, h, a.T0 + r, soff) + 8 * j;
  const void* base = kv ? a.v : a.k;
  float x[8];
  if (8 * j >= a.dh) {  // the padding of a head dim below D (a multiple of 8): zero pieces
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = 0.f;
  } else if constexpr (Q8) {
    const uint2 c = *reinterpret_cast<const uint2*>(reinterpret_cast<const char*>(base) + off);
    const float s = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(base) + soff);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      x[e] = (float)(int8_t)(((e < 4 ? c.x : c.y) >> (8 * (e & 3))) & 0xFF) * s;
  } else {
    const f32x4 x0 = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(base) + off);
    const f32x4 x1 = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(base) + off + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = x0[e];
      x[4 + e] = x1[e];
    }
  }
  auto row = [&](int p) { return out + ((((int64_t)kv * a.nkv + h) * 3 + p) * a.R + r) * D; };
  // two fp16 pieces of the row scaled by a power of two (split2h), the
  // row's unit (a float) at float r of the head's third piece
  uint32_t pc[2][4];
  float xm = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) xm = fmaxf(xm, fabsf(x[e]));
  xm = group_max<D / 8>(xm);  // the row's UPR lanes
  const int shift = kv ? f16_vrow_shift(xm) : f16_row_shift(xm);
#pragma unroll
  for (int e = 0; e < 8; e += 2) split2h(x[e], x[e + 1], shift, pc[0][e / 2], pc[1][e / 2]);
  if (j == 0)  // the units of a head's rows side by side in its third piece: row r's at float r
    reinterpret_cast<float*>(out + (((int64_t)kv * a.nkv + h) * 3 + 2) * a.R * D)[r] =
        kv ? f16_vrow_unit(xm, shift) : f16_row_unit(shift);
#pragma unroll
  for (int p = 0; p < 2; ++p)
    *reinterpret_cast<u32x4*>(row(p) + 8 * j) = u32x4{pc[p][0], pc[p][1], pc[p][2], pc[p][3]};
}

// One 16-byte global -> LDS copy per lane (global_load_lds_dwordx4, scalar
// base + lane offset): lane l's 16 bytes land at LDS address lds + 16*l.
// Written as inline assembly, so the compiler does not see an LDS store in
// flight: with the builtin it put an s_waitcnt vmcnt(0) before the next LDS
// reads it could not tell apart from the copy's destination (the transposed
// V reads of the other tile buffer), which waited for the next tile's copies
// halfway through every tile.  The kernel orders the copies itself
// (wait_vmcnt, then a barrier, before a buffer is read).  m0 takes the LDS
// address as an input operand (the compiler writes it); one wait state
// between that write and the copy.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(off), "s"(base), "{m0}"(lds)
               : "memory");
}
// The same with 4 bytes a lane (global_load_lds_dword): lane l's 4 bytes
// land at LDS address lds + 4*l.
__device__ __forceinline__ void dma4(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1"
               :
               : "v"(off), "s"(base), "{m0}"(lds)
               : "memory");
}

// Waves per prefill workgroup (16 query rows each): 8, so that 128 rows
// share each staged key tile and its split into pieces (32q/8kv/d128 fp32,
// 2048-token prompt: 285 -> 237 us).  fp32 pieces at d = 256 too (two
// waves a SIMD in 256 registers; 2048-token Gemma-style prompt: 127 ->
// 104 us, its grid then split over the keys).  A launch whose 8-wave grid
// would leave CUs idle and cannot be split takes 4 waves (512-token prompt
// after 16384 cached tokens: 1452 us on 8 waves, 1414 on 4).
constexpr int kPfWaves = 8;

// The kernel: every fp32 product is taken as 16-bit pieces on the dense
// matrix cores (16x the fp32 matrix rate).  Over fp32 and Q8 values both
// products take two fp16 pieces of each operand (split2h: hi = fp16(y),
// lo = fp16(y - hi) of y scaled by a power of two below 2^14) and three
// products (lo*hi, hi*lo, hi*hi) on v_mfma_f32_16x16x32_f16, the dropped
// lo*lo within 2^-22 of the term.  Scores: q and K rows scaled by their own
// powers of two, the score then times the two rows' units.  PV: V rows
// scaled the same way; each key's V unit folds into its p, and each query
// row's y = p * u_key stays below 2^14 through a running power of two that
// o carries (3 products a term instead of six bf16 ones: 2048-token prompt
// 194 -> 176 us with the scores' pieces, 173 -> 162 us with PV's).  A bf16
// cache needs one K/V piece (its values are exact) and q and P as three
// bf16 pieces (split3): three bf16 products each.  Tiles of 32 keys are
// staged into LDS as pieces:
//   K [KP][32 keys][D] 16-bit, 16-byte units XOR-swizzled by key (kt_off),
//     read as the A operand of S^T = K . Q^T: lane l key 16u + l%16,
//     elements 32s + 8(l/16) .. +7, Q^T in the same element order in
//     registers; fp32 and Q8 values: pieces 0 and 1 fp16 hi and lo, the
//     third slot the tile's 32 row units side by side (floats, f16_row_unit);
//   V [KP][32 keys][D] 16-bit, 16-byte units XOR-swizzled by key (vt_off),
//     read as V^T by ds_read_b64_tr_b16 as in attn_mfma_kernel: the A
//     operand of O^T += V^T . P^T, with P in the registers the score
//     accumulator left it in (key 16u + 4(l/16) + r of lane l, slot 4u + r);
//     fp32 and Q8 values as K (f16_vrow_unit).
// A tile's loads put keys 0..7 of one 16-byte column in lanes 0..7 and the
// next column in lanes 8..15 (128 contiguous bytes of each of 8 rows per 64
// lanes), so every LDS store of a piece is conflict-free too.
// D = 256 stages 100 KB (fp32 pieces) and runs one workgroup per CU.
template <int D, typename T, bool PAGED, int PW, bool PRE = false>
__global__ __launch_bounds__(64 * PW, PW == 4 && D < 256 ? 2 : 1)
void prefill_mfma16_kernel(PfArgs a) {
  static_assert(D == 64 || D == 128 || D == 256, "16-bit-piece prefill: D = 64, 128, 256");
  static_assert(PW == 4 || PW == 8, "4 or 8 waves");
  static_assert(!PRE || (sizeof(T) == 4 && !PAGED), "PRE: one instance per D and PW (pieces)");
  constexpr int NT = 64 * PW, QB = NT / 4;
  constexpr int KT = 32, KH = 2;
  constexpr int KP = sizeof(T) == 2 ? 1 : 3;  // staged pieces of K and V
  constexpr int KRB = 2 * D;                  // bytes of a staged K row
  constexpr int VRB = 2 * D;                  // bytes of a staged V row
  constexpr int QS = D / 32;                  // 32-element steps of the scores
  constexpr int DT = D / 16;
  constexpr int VW = KVT<T>::VW;              // elements per 16-byte load
  constexpr int CH = KT * D / VW;             // 16-byte chunks per tile (K or V)
  constexpr int CPT = (CH + NT - 1) / NT;
  constexpr bool Q8 = std::is_same<T, q8_t>::value;
  static_assert(CH % NT == 0 || CH < NT, "whole chunks per thread");
  static_assert((D / VW) % 4 == 0 && CH % 64 == 0 && 16 % VW == 0, "chunk mapping");
  // 8 waves (one workgroup a CU): two tile buffers where they fit, one
  // barrier a tile (a buffer is rewritten only after every wave has passed
  // the barrier that follows its last use); 4 waves: one buffer, so that two
  // workgroups share a CU's LDS
  constexpr int NBUF = PW == 8 && 2 * KP * KT * (KRB + VRB) <= 160 * 1024 ? 2 : 1;
  // KKV (pieces from the workspace, one buffer of each): a second K buffer
  // where it fits beside them, so that the next tile's K copies run under
  // the whole tile and its V copies under the next tile's scores
  constexpr bool KKV = PRE && NBUF == 1 && KP * KT * (2 * KRB + VRB) * (PW == 4 && D < 256 ? 2 : 1) <=
                                              160 * 1024;
  __shared__ __attribute__((aligned(16))) char kp_buf[KKV ? 2 : NBUF][KP * KT * KRB];
  __shared__ __attribute__((aligned(16))) char vp_buf[NBUF][KP * KT * VRB];

  const int G = a.nq / a.nkv;
  const int h = blockIdx.x % a.nkv;  // heads fastest: every XCD gets every head's share
  const int rest = (int)(blockIdx.x / a.nkv);
  const int sp = rest % a.nsplit;               // key split
  const int qb = a.nqb - 1 - rest / a.nsplit;  // latest rows (most keys) first
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, g4 = lane >> 4;
  const int rows = a.M * G;
  const int r0 = qb * QB;
  const int rl = min(r0 + QB, rows) - 1;
  auto t0_of = [&](int m) {
    const int pos = a.pos0 + m;
    int t0 = (a.window > 0 && pos - a.window + 1 > 0) ? pos - a.window + 1 : 0;
    return t0 > a.N ? a.N : t0;
  };
  auto nn_of = [&](int m) { return a.pos0 + m + 1 < a.N ? a.pos0 + m + 1 : a.N; };
  const int kt_lo = t0_of(r0 / G);
  const int kt_hi = nn_of(rl / G);
  const int ntile_all = kt_hi > kt_lo ? (kt_hi - kt_lo + KT - 1) / KT : 0;
  // this split's tiles [tb0, tb0 + ntile) of the block's range
  const int tb0 = (int)((int64_t)sp * ntile_all / a.nsplit);
  const int ntile = (int)((int64_t)(sp + 1) * ntile_all / a.nsplit) - tb0;
  const int kt_s = kt_lo + tb0 * KT;  // this split's first key
  const int row = r0 + 16 * w + c16;
  const bool rv = row < rows;
  const int m = rv ? row / G : 0;
  const int g = rv ? row - m * G : 0;
  const int rt0 = rv ? t0_of(m) : 0, rnn = rv ? nn_of(m) : 0;
  const int64_t qoff = ((int64_t)m * a.nq + h * G + g) * a.dh;  // q and O rows of dh elements

  // Q^T pieces (B operand): lane l row c16, elements 32s + 8*g4 + e, scaled
  // by scale*log2(e) (base-2 scores).  Against a bf16 cache (KP = 1, exact
  // K) three bf16 pieces; against fp32 and Q8 values (KP = 3) two fp16
  // pieces of the row scaled by a power of two (split2h; the row's 4 lanes
  // share its largest |q|), as K: three products per score term instead of
  // six bf16 ones, and the scores take the q and K row units back.
  const float qsc = a.scale * kLog2e;
  [[maybe_unused]] bf16x8_t qh[QS], qm[QS], ql[QS];
  [[maybe_unused]] f16x8_t fqh[QS], fql[QS];
  [[maybe_unused]] float qunit = 1.f;
  float qx[QS][8];
#pragma unroll
  for (int s = 0; s < QS; ++s) {
    const float* qp = a.q + qoff + 32 * s + 8 * g4;
    const bool qin = rv && 32 * s + 8 * g4 < a.dh;  // zero padding past dh (a multiple of 8)
    const f32x4 x0 = qin ? *reinterpret_cast<const f32x4*>(qp) : f32x4{0.f, 0.f, 0.f, 0.f};
    const f32x4 x1 = qin ? *reinterpret_cast<const f32x4*>(qp + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      qx[s][e] = x0[e] * qsc;
      qx[s][4 + e] = x1[e] * qsc;
    }
  }
  if constexpr (KP == 3) {
    float qm8 = 0.f;
#pragma unroll
    for (int s = 0; s < QS; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) qm8 = fmaxf(qm8, fabsf(qx[s][e]));
    const int qshift = f16_row_shift(max_xor32(max_xor16(qm8)));
    qunit = f16_row_unit(qshift);
#pragma unroll
    for (int s = 0; s < QS; ++s) {
      uint32_t h4[4], l4[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) split2h(qx[s][e], qx[s][e + 1], qshift, h4[e / 2], l4[e / 2]);
      fqh[s] = __builtin_bit_cast(f16x8_t, u32x4{h4[0], h4[1], h4[2], h4[3]});
      fql[s] = __builtin_bit_cast(f16x8_t, u32x4{l4[0], l4[1], l4[2], l4[3]});
    }
  } else {
#pragma unroll
    for (int s = 0; s < QS; ++s) {
      uint32_t h4[4], m4[4], l4[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) split3x2(qx[s][e], qx[s][e + 1], h4[e / 2], m4[e / 2], l4[e / 2]);
      qh[s] = __builtin_bit_cast(bf16x8_t, u32x4{h4[0], h4[1], h4[2], h4[3]});
      qm[s] = __builtin_bit_cast(bf16x8_t, u32x4{m4[0], m4[1], m4[2], m4[3]});
      ql[s] = __builtin_bit_cast(bf16x8_t, u32x4{l4[0], l4[1], l4[2], l4[3]});
    }
  }

  // tile loads: chunk c (16 bytes of the cache type) is key c%8 of its
  // key octet, column (c/8) % (D/VW) of the row, octet c / (8*D/VW).  KP = 3
  // (K split by rows, below): row-major, key c / (D/VW), column c % (D/VW),
  // so a row's D/VW chunks sit in consecutive lanes of one wave.
  constexpr int NCR = D / VW;  // chunks per row
  static_assert(KP != 3 || (NCR <= 64 && 64 % NCR == 0 && NT % NCR == 0), "rows within waves");
  auto chunk_of = [&](int c, int& key, int& e) {
    if constexpr (KP == 3) {
      key = c / NCR;
      e = VW * (c % NCR);
    } else {
      key = (c & 7) + 8 * (c / (8 * NCR));
      e = VW * ((c >> 3) % NCR);
    }
  };
  const T* Kb = reinterpret_cast<const T*>(a.k);
  const T* Vb = reinterpret_cast<const T*>(a.v);
  auto row_off = [&](int t, int64_t& soff) -> int64_t {
    return pf_row_off<D, T, PAGED>(a, h, t, soff);
  };
  // PRE: the tile's pieces straight from the split workspace into LDS, with
  // global_load_lds_dwordx4: lane l of a wave's load lands at the 16 bytes
  // base + 16*l of a 1 KB block (checked on the GPU), so lane l loads the
  // unit the swizzled layout keeps there (unit ch of key r at ch ^ f(r):
  // slot j holds unit j ^ f(r)).  No registers and no arithmetic per element.
  // The source is a wave-uniform row base (the tile's first key) plus a
  // 32-bit lane offset (key within the tile, clamped to the range's last
  // key, and its unit), so the loads take a scalar base and the per-tile
  // address arithmetic stays off the vector ALU.  The two pieces, then the
  // tile's 32 row units (128 bytes, dma4) to the start of the third piece
  // slot
  // (all 64 lanes: lanes 32..63 repeat the last key's unit into the unused
  // bytes 128..255 of the slot, so no lane is masked off)
  auto dunits = [&](int tk, char* buf, int kv) {
    const char* units = reinterpret_cast<const char*>(
        a.pieces + (((int64_t)kv * a.nkv + h) * 3 + 2) * a.R * D) + 4 * (int64_t)(tk - a.T0);
    const uint32_t lo = (uint32_t)(4 * min(min(lane, KT - 1), kt_hi - 1 - tk));
    dma4(units, lo, (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)(
                        buf + 2 * KT * (2 * D)));
  };
  auto dload = [&](int tk, char* kbuf, char* vbuf) {
    constexpr int UPR = D / 8;             // 16-byte units per row
    constexpr int KPB = 64 / UPR;          // keys per 1 KB block
    constexpr int BPP = KT / KPB;          // blocks per piece
    constexpr int NBL = 2 * 2 * BPP;       // blocks per tile (K, V; 2 pieces)
    const int r_in = lane / UPR, jpos = lane % UPR;
    const int lastr = kt_hi - 1 - tk;      // the range's last key, from the tile's first
    if (w < 2) dunits(tk, w ? vbuf : kbuf, w);
#pragma unroll
    for (int bi0 = 0; bi0 < NBL; bi0 += PW) {
      const int bi = bi0 + w;  // wave-uniform
      if (NBL % PW != 0 && bi >= NBL) break;
      const int kv = bi / (2 * BPP), rem = bi - kv * 2 * BPP;
      const int pc = rem / BPP, kb = rem - pc * BPP;
      const int r = kb * KPB + r_in;
      const int ch = jpos ^ (kv ? vt_f<D>(r) : kt_f<D>(r));
      const char* rows = reinterpret_cast<const char*>(
          a.pieces + ((((int64_t)kv * a.nkv + h) * 3 + pc) * a.R + (tk - a.T0)) * D);
      const uint32_t lo = (uint32_t)(min(r, lastr) * (2 * D) + 16 * ch);
      char* dst = (kv ? vbuf : kbuf) + pc * KT * (2 * D) + kb * 1024;
      dma16(rows, lo, (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)dst);
    }
  };
  // K (kv = 0) or V (kv = 1) of a tile alone: NL copies a wave (every wave
  // copies the units, the same bytes to the same place, so that the waves
  // count alike)
  constexpr int NL = 2 * (KT / (64 / (D / 8))) / PW + 1;
  auto dload1 = [&](int tk, char* buf, int kv) {
    constexpr int UPR = D / 8, KPB = 64 / UPR, BPP = KT / KPB;
    static_assert(!KKV || (2 * BPP) % PW == 0, "the same copies in every wave");
    const int r_in = lane / UPR, jpos = lane % UPR;
    const int lastr = kt_hi - 1 - tk;
    dunits(tk, buf, kv);
#pragma unroll
    for (int bi0 = 0; bi0 < 2 * BPP; bi0 += PW) {
      const int bi = bi0 + w;  // wave-uniform
      const int pc = bi / BPP, kb = bi - pc * BPP;
      const int r = kb * KPB + r_in;
      const int ch = jpos ^ (kv ? vt_f<D>(r) : kt_f<D>(r));
      const char* rows = reinterpret_cast<const char*>(
          a.pieces + ((((int64_t)kv * a.nkv + h) * 3 + pc) * a.R + (tk - a.T0)) * D);
      const uint32_t lo = (uint32_t)(min(r, lastr) * (2 * D) + 16 * ch);
      char* dst = buf + pc * KT * (2 * D) + kb * 1024;
      dma16(rows, lo, (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)dst);
    }
  };
  typename KVT<T>::vec kreg[CPT], vreg[CPT];
  [[maybe_unused]] float ksc[CPT], vsc[CPT];
  auto load_tile = [&](int tk) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + NT * i;
      if (CH < NT && c >= CH) break;
      int key, e;
      chunk_of(c, key, e);
      const int t = min(tk + key, kt_hi - 1);  // rows past the range: the last one (masked)
      int64_t soff = 0;
      const int64_t off = row_off(t, soff) + e;
      if constexpr (Q8) {
        ksc[i] = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(a.k) + soff);
        vsc[i] = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(a.v) + soff);
      }
      if (e < a.dh) {  // a padded launch: columns past the stored head dim read as 0
        kreg[i] = load16(Kb + off);
        vreg[i] = load16(Vb + off);
      } else {
        kreg[i] = typename KVT<T>::vec{};
        vreg[i] = typename KVT<T>::vec{};
      }
    }
  };
  // the chunk's values as KP pieces (K of fp32 and Q8 values: two fp16 of
  // the row scaled by a power of two, its unit in the third), 4 elements
  // (8 bytes) at a time
  auto store_tile = [&](char* kp_s, char* vp_s) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + NT * i;
      if (CH < NT && c >= CH) break;
      int key, e;
      chunk_of(c, key, e);
      float kx[VW], vx[VW];
      KVT<T>::unpack(kreg[i], kx);
      KVT<T>::unpack(vreg[i], vx);
      if constexpr (Q8) {  // code * s, the dequantized value
#pragma unroll
        for (int j = 0; j < VW; ++j) {
          kx[j] *= ksc[i];
          vx[j] *= vsc[i];
        }
      }
      [[maybe_unused]] int kshift = 0, vshift = 0;
      if constexpr (KP == 3) {  // the K and V rows' scales: largest |x| over the row's NCR lanes
        float km = 0.f, vm = 0.f;
#pragma unroll
        for (int j = 0; j < VW; ++j) {
          km = fmaxf(km, fabsf(kx[j]));
          vm = fmaxf(vm, fabsf(vx[j]));
        }
        kshift = f16_row_shift(group_max<NCR>(km));
        vm = group_max<NCR>(vm);
        vshift = f16_vrow_shift(vm);
        if (e == 0) {  // the tile's row units side by side in the third slot
          reinterpret_cast<float*>(kp_s + 2 * KT * KRB)[key] = f16_row_unit(kshift);
          reinterpret_cast<float*>(vp_s + 2 * KT * VRB)[key] = f16_vrow_unit(vm, vshift);
        }
      }
#pragma unroll
      for (int j4 = 0; j4 < VW; j4 += 4) {
        const int ej = e + j4;
        uint32_t kpc[KP][2], vpc[KP][2];  // 4 elements of each piece
#pragma unroll
        for (int j = 0; j < 4; j += 2) {
          if constexpr (KP == 3) {
            split2h(kx[j4 + j], kx[j4 + j + 1], kshift, kpc[0][j / 2], kpc[1][j / 2]);
            split2h(vx[j4 + j], vx[j4 + j + 1], vshift, vpc[0][j / 2], vpc[1][j / 2]);
          } else {  // exact bf16 values
            kpc[0][j / 2] = bf16_pair(kx[j4 + j], kx[j4 + j + 1]);
            vpc[0][j / 2] = bf16_pair(vx[j4 + j], vx[j4 + j + 1]);
          }
        }
        const int kofs = kt_off<D>(key, ej >> 3) + 8 * ((ej >> 2) & 1);
        const int vofs = vt_off<D>(key, ej >> 3) + 8 * ((ej >> 2) & 1);
#pragma unroll
        for (int p = 0; p < (KP == 3 ? 2 : 1); ++p) {  // the third piece holds the row's unit only
          *reinterpret_cast<u32x2*>(kp_s + p * KT * KRB + kofs) = u32x2{kpc[p][0], kpc[p][1]};
          *reinterpret_cast<u32x2*>(vp_s + p * KT * VRB + vofs) = u32x2{vpc[p][0], vpc[p][1]};
        }
      }
    }
  };

  f32x4 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  // scores of the two 16-key halves of the tile at kp_s, smallest piece
  // products first; even and odd 32-element steps into separate
  // accumulators (four independent MFMA chains, added at the end)
  // piece products in the order they enter an accumulator, smallest first:
  // (K or V piece, q or P piece: 0 hi, 1 mid, 2 lo)
  constexpr int NPR = KP == 3 ? 6 : 3;
  // 32-element steps whose operands are read together, and 16-row V blocks
  // (d = 256: fewer, to stay in 256 registers)
  constexpr int SJ = D == 256 ? 1 : 2;
  constexpr int NDT = D == 256 ? 2 : (DT >= 4 ? 4 : DT);
  constexpr int PRK[6] = {KP == 3 ? 1 : 0, KP == 3 ? 2 : 0, 0, 1, 0, 0};
  constexpr int PRQ[6] = {KP == 3 ? 1 : 2, KP == 3 ? 0 : 1, KP == 3 ? 2 : 0, 0, 1, 0};
  // scores of the two 16-key halves of the tile at kp_s.  SJ 32-element
  // steps at a time: their staged K operands (both halves, every piece) are
  // read first, then the piece products go out piece by piece across the
  // accumulators (even and odd steps of each half), so that consecutive
  // matrix instructions are independent; each accumulator takes its
  // products in the same order as one at a time.  The two step parities are
  // added at the end.
  // KP = 3 (fp32 and Q8 values): K and q as two fp16 pieces each, three
  // products per term (lo*hi, hi*lo, hi*hi; the dropped lo*lo is within
  // 2^-22 of the term), then the q and K row units multiply each score.
  constexpr int FPK[3] = {1, 0, 0};
  constexpr int FPQ[3] = {0, 1, 0};
  auto scores = [&](const char* kp_s, f32x4 (&sacc)[KH]) {
    f32x4 sacc2[KH][2];
#pragma unroll
    for (int u = 0; u < KH; ++u) sacc2[u][0] = sacc2[u][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s0 = 0; s0 < QS; s0 += SJ) {
      if constexpr (KP == 3) {
        f16x8_t kk[SJ][KH][2];
#pragma unroll
        for (int j = 0; j < SJ; ++j)
#pragma unroll
          for (int u = 0; u < KH; ++u) {
            const char* kb = kp_s + kt_off<D>(16 * u + c16, 4 * (s0 + j) + g4);
#pragma unroll
            for (int p = 0; p < 2; ++p)
              kk[j][u][p] = *reinterpret_cast<const f16x8_t*>(kb + p * KT * KRB);
          }
#pragma unroll
        for (int t = 0; t < 3; ++t)
#pragma unroll
          for (int j = 0; j < SJ; ++j)
#pragma unroll
            for (int u = 0; u < KH; ++u) {
              f32x4& acc = sacc2[u][(s0 + j) & 1];
              acc = mfma_f16(kk[j][u][FPK[t]], FPQ[t] == 0 ? fqh[s0 + j] : fql[s0 + j], acc);
            }
      } else {
        bf16x8_t kk[SJ][KH][KP];
#pragma unroll
        for (int j = 0; j < SJ; ++j)
#pragma unroll
          for (int u = 0; u < KH; ++u) {
            const char* kb = kp_s + kt_off<D>(16 * u + c16, 4 * (s0 + j) + g4);
#pragma unroll
            for (int p = 0; p < KP; ++p)
              kk[j][u][p] = *reinterpret_cast<const bf16x8_t*>(kb + p * KT * KRB);
          }
#pragma unroll
        for (int t = 0; t < NPR; ++t)
#pragma unroll
          for (int j = 0; j < SJ; ++j)
#pragma unroll
            for (int u = 0; u < KH; ++u) {
              const bf16x8_t& qp = PRQ[t] == 0 ? qh[s0 + j] : PRQ[t] == 1 ? qm[s0 + j] : ql[s0 + j];
              f32x4& acc = sacc2[u][(s0 + j) & 1];
              acc = mfma_bf16(kk[j][u][PRK[t]], qp, acc);
            }
      }
    }
#pragma unroll
    for (int u = 0; u < KH; ++u) sacc[u] = sacc2[u][0] + sacc2[u][1];
    if constexpr (KP == 3) {
      // keys 16u + 4*g4 .. +3's units: floats 16u + 4*g4 .. of the third slot
      // (the q row's unit, the same for the row's every score, is the
      // softmax's: its max and exponent arguments take it)
#pragma unroll
      for (int u = 0; u < KH; ++u) {
        const f32x4 ku = *reinterpret_cast<const f32x4*>(kp_s + 2 * KT * KRB + 4 * (16 * u + 4 * g4));
#pragma unroll
        for (int r = 0; r < 4; ++r) sacc[u][r] *= ku[r];
      }
    }
  };
  // online softmax (base 2) of this lane's row over its 8 keys of the tile
  // at tk.  Lazy rescale, as in the decode kernel: the running max moves
  // only when a score exceeds it by more than kLazyMax (p <= 2^8 otherwise);
  // o and l always share the max they were formed with.  Leaves P^T (the
  // B operand's order: pv[4u + r] is key 16u + 4*g4 + r), the factor alpha
  // that o and l take before P is added (1 unless the max moved) and the
  // tile's row sum.
  // FULL (a std::integral_constant): every key of the tile is in every
  // row's range, so no key is masked and every probability is an exp.
  auto softmax = [&](auto FULL, const f32x4 (&sacc)[KH], int tk, float (&pv)[4 * KH],
                     float& alpha, bool& grow, int& gsh, float& ps) {
    constexpr bool full = decltype(FULL)::value;
    float sv[KH][4];
    float tmax = -INFINITY;
#pragma unroll
    for (int u = 0; u < KH; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = tk + 16 * u + 4 * g4 + r;
        sv[u][r] = (full || (t >= rt0 && t < rnn)) ? sacc[u][r] : -INFINITY;
        tmax = fmaxf(tmax, sv[u][r]);
      }
    // the scores over fp32 and Q8 values still lack the q row's unit qunit
    // (a power of two): tmax takes it, and each exponent argument as one fma,
    // s * qunit - m, rounded once as the difference of the scaled score was
    tmax = max_xor32(max_xor16(tmax)) * qunit;
    grow = tmax > m_run + kLazyMax;  // false while the row has no key (-inf)
    const float mn = grow ? fmaxf(m_run, tmax) : m_run;
    alpha = m_run == -INFINITY ? 1.f : exp2_hw(m_run - mn);  // exp2(0) = 1 exactly
    // floor(log2(1 / alpha)) (> 8, at most 1000) when a finite max moved
    gsh = (grow && m_run != -INFINITY) ? (int)fminf(floorf(mn - m_run), 1000.f) : 0;
    m_run = mn;
    ps = 0.f;
#pragma unroll
    for (int u = 0; u < KH; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pv[4 * u + r] =
            (!full && sv[u][r] == -INFINITY) ? 0.f : exp2_hw(fmaf(sv[u][r], qunit, -m_run));
        ps += pv[4 * u + r];
      }
  };
  // V^T of the 16-row blocks dt0 .. dt0 + NDT - 1 (A operands of PV), piece
  // p of the staged tile at vp_s: two transposed reads per block
  auto read_vt = [&](const char* vp_s, int dt0, int p, auto& av) {
#pragma unroll
    for (int j = 0; j < NDT; ++j) {
      i16x4_t t2[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int r = (lane >> 2) + 16 * u;
        t2[u] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4_t*)(
                vp_s + p * KT * VRB + vt_off<D>(r, 2 * (dt0 + j) + ((lane & 3) >> 1)) +
                8 * (lane & 1)));
      }
      av[j][p] = __builtin_bit_cast(typename std::remove_reference<decltype(av[j][p])>::type,
                                    __builtin_shufflevector(t2[0], t2[1], 0, 1, 2, 3, 4, 5, 6, 7));
    }
  };
  // fp32 and Q8 values (KP = 3): PV takes y = p * u_key * 2^wsh as two fp16
  // pieces, u_key the key's V row unit (V's pieces are the row over u_key),
  // so that o = 2^wsh * sum p v.  wsh (per query row: this lane's column of
  // O^T) keeps y below 2^14: it follows the largest p * u_key of the row's
  // keys so far, and when the running max moves (o and l scaled by alpha)
  // it may grow by floor(log2(1 / alpha)), so that the unit follows o down.
  // Each term is then held to 2^-22 of itself, or to 2^-25 of the
  // row's unit 2^(14 - wsh) (2^-37 of its largest p * |v| term) below.
  constexpr int kNoShift = 1 << 20;  // no key yet (o = 0)
  [[maybe_unused]] int wsh = kNoShift;
  // o += P V over the tile at vp_s.  bf16 caches (exact V): P as three bf16
  // pieces, V^T of NDT 16-row blocks at a time, their operands first, then
  // the piece products piece by piece across the NDT accumulators (each in
  // the same order as one block at a time).  fp32 and Q8 values: y and V as
  // two fp16 pieces each, three products per term (lo*hi, hi*lo, hi*hi; the
  // dropped lo*lo is within 2^-22 of the term), as the scores.  gsh: the
  // softmax's floor(log2(1 / alpha)) when the running max moved, else 0.
  auto pv_acc = [&](const char* vp_s, const float (&pv)[4 * KH], int gsh) {
    if constexpr (KP == 3) {
      float z[4 * KH];  // p * u_key, u_key from the tile's units in the third slot
      float zt = 0.f;
#pragma unroll
      for (int u = 0; u < KH; ++u) {
        const f32x4 uk = *reinterpret_cast<const f32x4*>(vp_s + 2 * KT * VRB + 4 * (16 * u + 4 * g4));
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          z[4 * u + r] = pv[4 * u + r] * uk[r];
          zt = fmaxf(zt, z[4 * u + r]);
        }
      }
      zt = max_xor32(max_xor16(zt));  // the row's 32 keys (its column's 4 lanes)
      const int ns = min(min(wsh + gsh, kNoShift), zt > 0.f ? f16_row_shift(zt) : kNoShift);
      if (__builtin_amdgcn_ballot_w64(ns != wsh) != 0) {  // o into the new unit (exact)
        const int dsh = ns - wsh;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int i = 0; i < 4; ++i) o[dt][i] = ldexpf(o[dt][i], dsh);
      }
      wsh = ns;
      uint32_t h4[4], l4[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) split2h(z[e], z[e + 1], ns, h4[e / 2], l4[e / 2]);
      const f16x8_t yh = __builtin_bit_cast(f16x8_t, u32x4{h4[0], h4[1], h4[2], h4[3]});
      const f16x8_t yl = __builtin_bit_cast(f16x8_t, u32x4{l4[0], l4[1], l4[2], l4[3]});
#pragma unroll
      for (int dt0 = 0; dt0 < DT; dt0 += NDT) {
        f16x8_t av[NDT][2];
        read_vt(vp_s, dt0, 0, av);
        read_vt(vp_s, dt0, 1, av);
#pragma unroll
        for (int t = 0; t < 3; ++t)
#pragma unroll
          for (int j = 0; j < NDT; ++j)
            o[dt0 + j] = mfma_f16(av[j][FPK[t]], FPQ[t] == 0 ? yh : yl, o[dt0 + j]);
      }
    } else {
      uint32_t ph4[4], pm4[4], pl4[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) split3x2(pv[e], pv[e + 1], ph4[e / 2], pm4[e / 2], pl4[e / 2]);
      const bf16x8_t ph = __builtin_bit_cast(bf16x8_t, u32x4{ph4[0], ph4[1], ph4[2], ph4[3]});
      const bf16x8_t pm = __builtin_bit_cast(bf16x8_t, u32x4{pm4[0], pm4[1], pm4[2], pm4[3]});
      const bf16x8_t pl = __builtin_bit_cast(bf16x8_t, u32x4{pl4[0], pl4[1], pl4[2], pl4[3]});
#pragma unroll
      for (int dt0 = 0; dt0 < DT; dt0 += NDT) {
        bf16x8_t av[NDT][KP];
#pragma unroll
        for (int p = 0; p < KP; ++p) read_vt(vp_s, dt0, p, av);
#pragma unroll
        for (int t = 0; t < NPR; ++t)
#pragma unroll
          for (int j = 0; j < NDT; ++j) {
            const bf16x8_t& pp = PRQ[t] == 0 ? ph : PRQ[t] == 1 ? pm : pl;
            o[dt0 + j] = mfma_bf16(av[j][PRK[t]], pp, o[dt0 + j]);
          }
      }
    }
  };
  // o and l take alpha, then l the tile's sum (two roundings, as the
  // running sums of the decode kernels)
  auto rescale = [&](float alpha, bool grow, float ps) {
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
    }
    {
#pragma clang fp contract(off)
      l_run = l_run * alpha + ps;
    }
  };

  if constexpr (KKV) {
    // Iteration it: the scores read K(it) while K(it+1) is copied into the
    // other K buffer (last read by the scores of it-1, before the barrier
    // that ended it-1); PV reads V(it), copied at the end of it-1 under the
    // scores and softmax of it; V(it+1) is copied once every wave is past
    // PV(it).  Each wave counts its own copies: NL for K or V of a tile.
    if (ntile > 0) {
      dload(kt_s, kp_buf[0], vp_buf[0]);
      wait_vmcnt<0>();
      __syncthreads();
    }
    for (int it = 0; it < ntile; ++it) {
      const int tk = kt_s + it * KT;
      const bool more = it + 1 < ntile;
      if (more) dload1(tk + KT, kp_buf[(it + 1) & 1], 0);
      f32x4 sacc[KH];
      scores(kp_buf[it & 1], sacc);
      float pv[4 * KH];
      float alpha, ps;
      bool grow;
      int gsh;
      if (__builtin_amdgcn_ballot_w64(!(rv && tk >= rt0 && tk + KT <= rnn)) == 0)
        softmax(std::true_type{}, sacc, tk, pv, alpha, grow, gsh, ps);
      else
        softmax(std::false_type{}, sacc, tk, pv, alpha, grow, gsh, ps);
      rescale(alpha, grow, ps);
      // V(it) is in LDS (K(it+1), copied after it, may still be in flight)
      if (more)
        wait_vmcnt<NL>();
      else
        wait_vmcnt<0>();
      lds_barrier();
      pv_acc(vp_buf[0], pv, gsh);
      if (more) {
        lds_barrier();  // every wave is past PV(it)
        dload1(tk + KT, vp_buf[0], 1);
        wait_vmcnt<NL>();  // K(it+1) is in LDS (V(it+1) may still be in flight)
        lds_barrier();
      }
    }
  } else {
    if constexpr (PRE) {
      if (ntile > 0) dload(kt_s, kp_buf[0], vp_buf[0]);
      wait_vmcnt<0>();  // this wave's direct loads are in LDS
      __syncthreads();
    } else {
      if (ntile > 0) load_tile(kt_s);
    }
    for (int it = 0; it < ntile; ++it) {
      const int tk = kt_s + it * KT;
      const int bf = NBUF == 2 ? (it & 1) : 0;
      const char* kp_s = kp_buf[bf];
      const char* vp_s = vp_buf[bf];
      if constexpr (PRE) {
        // the other buffer was last read in the previous tile, which every
        // wave finished before the barrier that ended it
        if constexpr (NBUF == 2)
          if (it + 1 < ntile) dload(tk + KT, kp_buf[bf ^ 1], vp_buf[bf ^ 1]);
      } else {
        store_tile(kp_buf[bf], vp_buf[bf]);
        __syncthreads();
        if (it + 1 < ntile) load_tile(tk + KT);  // in flight while this tile is used
      }
      f32x4 sacc[KH];
      scores(kp_s, sacc);
      float pv[4 * KH];
      float alpha, ps;
      bool grow;
      int gsh;
      // interior tile: every row of the wave attends all of its keys
      if (__builtin_amdgcn_ballot_w64(!(rv && tk >= rt0 && tk + KT <= rnn)) == 0)
        softmax(std::true_type{}, sacc, tk, pv, alpha, grow, gsh, ps);
      else
        softmax(std::false_type{}, sacc, tk, pv, alpha, grow, gsh, ps);
      rescale(alpha, grow, ps);
      pv_acc(vp_s, pv, gsh);
      if constexpr (PRE) {
        if constexpr (NBUF == 1) {
          __syncthreads();  // every wave is done with the buffer
          if (it + 1 < ntile) dload(tk + KT, kp_buf[0], vp_buf[0]);
        }
        wait_vmcnt<0>();  // this wave's direct loads of the next tile are in LDS
        __syncthreads();
      } else {
        if constexpr (NBUF == 1) __syncthreads();  // the tile's LDS is rewritten next
      }
    }
  }
  l_run = sum_xor32(sum_xor16(l_run));
  if constexpr (KP == 3) {  // o back from 2^wsh * sum p v (a power of two; no key: o = 0)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[dt][i] = ldexpf(o[dt][i], -wsh);
  }
  if (rv && a.nsplit > 1) {  // the split's partial: unnormalised o, max in natural units, sum
    const int64_t ps = ((int64_t)m * a.nq + h * G + g) * a.nsplit + sp;
    float* po = a.part_o + ps * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<f32x4*>(po + 16 * dt + 4 * g4) = o[dt];
    if (g4 == 0) {
      a.part_ml[2 * ps] = m_run == -INFINITY ? -INFINITY : m_run * kLn2;
      a.part_ml[2 * ps + 1] = l_run;
    }
  } else if (rv) {
    const float inv = l_run > 0.f ? 1.f / l_run : 0.f;  // no key: O = 0 (gemm.h:438)
    float* orow = a.o + qoff;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      if (16 * dt + 4 * g4 < a.dh) *reinterpret_cast<f32x4*>(orow + 16 * dt + 4 * g4) = o[dt] * inv;
  }
}

// Log-sum-exp combine of the chunk partials of split-K launches.  Grid
// (slots, P/pairs), the slot fastest: workgroup id % 8 is the XCD, so where
// the attention launch ran a slot's chunks on XCD slot % 8 (its slot index
// fastest over a multiple of 8 slots) the combine reads their partials from
// that XCD's L2 (32q/8kv/d128 fp32 at n = 4097: step 12.8 -> 12.1 us).  A
// workgroup takes `pairs` output pairs of one head of a
// slot (pairs divides D) with 256/pairs threads per pair, thread phase ph
// folding chunks ph, ph + phases, ...  The chunk weights e^(m_c - M) and the
// sum L are computed once per workgroup into LDS; the first round of o
// loads is issued before that, so a whole combine costs about one memory
// round trip when phases * kCombRound covers the chunks (comb_pairs picks
// the pairs so: 64 pairs of 4 phases up to 32 chunks, 16 pairs of 16 phases
// from 65).  Slots whose sequence has a single chunk were written by the
// attention kernel itself.
struct CombArgs {
  const float* part_o;
  const float* part_ml;
  const float* qrot;
  float* o;
  float* q_out;
  const int32_t* seq_lens;
  const int32_t* pos_arr;
  int nq, nkv, gh, nsub, d, nchunks, chunk, window, rope, paged;
  int fold;  // the attention launch folded in a new token (its chunks tile n - 1 rows)
  int dh;    // head dim as stored (d: the partials' padded head dim)
  int pf, pos0, n;  // prefill rows (AttnArgs::pf): row b at pos0 + b of a cache of n rows
  int pairs;        // combine_kernel: output pairs per workgroup (16, 32 or 64)
};

// Chunks of sequence b of a per-sequence launch (a paged batch, or prefill
// rows), as the attention kernel derives them.
__device__ __forceinline__ int comb_chunks(const CombArgs& a, int b) {
  int n, pos;
  if (a.pf) {
    pos = a.pos0 + b;
    n = pos + 1 < a.n ? pos + 1 : a.n;
  } else {
    n = a.seq_lens[b];
    pos = a.pos_arr ? a.pos_arr[b] : n - 1;
  }
  int t0 = (a.window > 0 && pos - a.window + 1 > 0) ? pos - a.window + 1 : 0;
  if (t0 > n) t0 = n;
  const int span = (a.fold ? n - 1 : n) - t0;
  const int nch = span > 0 ? (span + a.chunk - 1) / a.chunk : (a.fold ? 1 : 0);
  return nch > a.nchunks ? a.nchunks : nch;
}

constexpr int kCombThreads = 256;
constexpr int kCombPairs = 64;                          // most pairs per workgroup
constexpr int kCombRound = 8;                           // o loads in flight per thread

// Pairs per combine workgroup for nch chunks: the fewest phases (threads per
// pair) whose one round of kCombRound loads each covers the chunks, at most
// 16 (8q/2kv/d512, 128 chunks per KV head: 6.2 us on 64 pairs of 4 phases).
__host__ __device__ constexpr int comb_pairs(int nch) {
  int ph = 4;
  while (ph < 16 && ph * kCombRound < nch) ph *= 2;
  return kCombThreads / ph;
}
constexpr int kMaxChunks = 4096;

// LDS of one combine workgroup, in floats: the chunk weights and sums of
// the launch's chunk count, the phases' partial sums and L.
__host__ __device__ constexpr int comb_lds_floats(int nchunks) { return 2 * nchunks + kCombThreads + 4; }

__global__ __launch_bounds__(kCombThreads) void combine_kernel(CombArgs a) {
  extern __shared__ float csm[];
  float* wts = csm;                  // [nchunks] m_c, then the chunk weight e^(m_c - M)
  float* lsv = csm + a.nchunks;      // [nchunks] l_c
  float* pacc = lsv + a.nchunks;     // [kCombThreads]
  float& s_l = pacc[kCombThreads];   // L = sum_c e^(m_c - M) l_c
  const int P = a.gh * a.d;
  const int slot = blockIdx.x;
  const int pairs = a.pairs, phases = kCombThreads / pairs;
  const int pb = blockIdx.y * pairs;
  const int t = threadIdx.x;
  const int rows = a.nkv * a.nsub;  // slots per sequence
  const int b = slot / rows, y = slot - b * rows;
  const int pl = t % pairs, ph = t / pairs;
  const int pair = pb + pl;  // < P: P is a multiple of 64
  const int g = pb / a.d;    // one head per workgroup
  const float* po = a.part_o + (int64_t)slot * a.nchunks * P + pair;
  const float* pml = a.part_ml + (int64_t)slot * a.nchunks * a.gh * 2 + 2 * g;
  // The first round of o loads and wave 0's first statistics go out before
  // this sequence's chunk count is known (paged: it needs seq_lens, another
  // round trip): they stay within the launch's nchunks slots of the
  // workspace, and only chunks below the count are used.
  float ov[kCombRound];
#pragma unroll
  for (int u = 0; u < kCombRound; ++u)
    ov[u] = po[(int64_t)min(ph + phases * u, a.nchunks - 1) * P];
  float m1 = -INFINITY, l1 = 0.f;
  if (t < 64) {
    const int c1 = min(t, a.nchunks - 1);
    m1 = pml[(int64_t)c1 * a.gh * 2];
    l1 = pml[(int64_t)c1 * a.gh * 2 + 1];
  }
  // this sequence's chunk count, as the attention kernel derives it
  const int nch = a.paged || a.pf ? comb_chunks(a, b) : a.nchunks;
  if (nch <= 1) return;  // uniform over the workgroup
  if (t < 64) {  // wave 0: chunk weights and L of head g
    float mloc = -INFINITY;
    for (int cc = t; cc < nch; cc += 64) {
      const float m = cc == t ? m1 : pml[(int64_t)cc * a.gh * 2];
      wts[cc] = m;
      lsv[cc] = cc == t ? l1 : pml[(int64_t)cc * a.gh * 2 + 1];
      mloc = fmaxf(mloc, m);
    }
    const float M = wave_reduce<true>(mloc);
    float lloc = 0.f;
    for (int cc = t; cc < nch; cc += 64) {  // the lane's own LDS entries
      // a prefill row no split attended: M = -inf, weights 0, O = 0 below
      const float wgt = M == -INFINITY ? 0.f : softmax_exp(wts[cc] - M);
      wts[cc] = wgt;
      lloc = fmaf(wgt, lsv[cc], lloc);
    }
    const float Ls = wave_reduce<false>(lloc);
    if (t == 0) s_l = Ls;
  }
  __syncthreads();
  float acc = 0.f;
#pragma unroll
  for (int u = 0; u < kCombRound; ++u) {
    const int cc = ph + phases * u;
    if (cc < nch) acc = fmaf(wts[cc], ov[u], acc);
  }
  for (int c0 = ph + phases * kCombRound; c0 < nch; c0 += phases * kCombRound) {
#pragma unroll
    for (int u = 0; u < kCombRound; ++u)
      ov[u] = po[(int64_t)min(c0 + phases * u, nch - 1) * P];
#pragma unroll
    for (int u = 0; u < kCombRound; ++u) {
      const int cc = c0 + phases * u;
      if (cc < nch) acc = fmaf(wts[cc], ov[u], acc);
    }
  }
  pacc[t] = acc;
  __syncthreads();
  if (ph == 0) {
    float o = acc;
    for (int q2 = 1; q2 < phases; ++q2) o += pacc[q2 * pairs + pl];
    const int G = a.nq / a.nkv;
    const int h = y / a.nsub, sub = y - h * a.nsub;
    const int64_t oi = out_index((int64_t)b * a.nq + h * G + sub * a.gh, pair, a.d, a.dh);
    if (oi >= 0) {
      a.o[oi] = s_l > 0.f ? o / s_l : 0.f;
      if (a.rope && a.q_out) a.q_out[oi] = a.qrot[(int64_t)slot * P + pair];
    }
  }
}

// The merge for a few chunks per slot (R >= nchunks, R <= 64), one wave per
// 64 output pairs of one head, with no LDS and no barrier: lane c holds chunk c's (m, l), DPP
// reductions give the max M and L = sum_c e^(m_c - M) l_c, and every lane
// sums its pair over the chunks with the weights broadcast by readlane.
// All R >= nchunks o loads and the statistics go out at once, before this
// sequence's chunk count is known (paged: it needs seq_lens): they stay
// within the launch's nchunks slots of the workspace, and only chunks below
// the count are used.  Grid (slots, P/threads), the slot fastest, as
// combine_kernel's.
constexpr int kCombWaveThreads = 256;
template <int R>
__global__ __launch_bounds__(kCombWaveThreads) void combine_wave_kernel(CombArgs a) {
  const int P = a.gh * a.d;
  const int slot = blockIdx.x;
  const int pair = blockIdx.y * blockDim.x + threadIdx.x;  // < P: blockDim divides P
  const int lane = threadIdx.x & 63;
  const int g = __builtin_amdgcn_readfirstlane(pair / a.d);  // d % 64 == 0: one head per wave
  const int rows = a.nkv * a.nsub;  // slots per sequence
  const int b = slot / rows, y = slot - b * rows;
  const float* po = a.part_o + (int64_t)slot * a.nchunks * P + pair;
  const float* pml = a.part_ml + (int64_t)slot * a.nchunks * a.gh * 2 + 2 * g;
  float ov[R];
#pragma unroll
  for (int u = 0; u < R; ++u) ov[u] = po[(int64_t)min(u, a.nchunks - 1) * P];
  const int cl = min(lane, a.nchunks - 1);
  const float mc = pml[(int64_t)cl * a.gh * 2], lc = pml[(int64_t)cl * a.gh * 2 + 1];
  // this sequence's chunk count, as the attention kernel derives it
  const int nch = a.paged || a.pf ? comb_chunks(a, b) : a.nchunks;
  if (nch <= 1) return;  // uniform over the workgroup
  const bool live = lane < nch;
  const float M = wave_reduce<true>(live ? mc : -INFINITY);
  // a slot whose chunks all saw no key (max -inf) gets O = 0, as in combine_kernel
  const float wc = live && M != -INFINITY ? softmax_exp(mc - M) : 0.f;
  const float L = wave_reduce<false>(live ? wc * lc : 0.f);
  float acc = 0.f;
#pragma unroll
  for (int u = 0; u < R; ++u)
    if (u < nch) acc = fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(wc), u)), ov[u], acc);
  const int G = a.nq / a.nkv;
  const int h = y / a.nsub, sub = y - h * a.nsub;
  const int64_t oi = out_index((int64_t)b * a.nq + h * G + sub * a.gh, pair, a.d, a.dh);
  if (oi >= 0) {
    a.o[oi] = L > 0.f ? acc / L : 0.f;
    if (a.rope && a.q_out) a.q_out[oi] = a.qrot[(int64_t)slot * P + pair];
  }
}

// The prefill's key-split merge: slot s = (token, q head) of one head, P = D
// partial outputs over R >= nchunks splits.  A wave takes 64V consecutive
// outputs of one slot (V = 4 at D % 256 == 0, 2 at D % 128 == 0, else 1), so
// a 2048-token prompt of 8 q heads at d = 256 runs 16384 waves instead of
// 65536; the arithmetic and its order are combine_wave_kernel's (lane c
// holds split c's (m, l), DPP reductions give M and L, the weights reach
// every lane by readlane), so the outputs are the same bits.  Four waves a
// workgroup, consecutive units (slot, 64V-span); units past the last exit.
template <int V>
__device__ __forceinline__ void load_v(const float* p, float* x) {
  if constexpr (V == 4) {
    const f32x4 t = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = t[e];
  } else if constexpr (V == 2) {
    const f32x2 t = *reinterpret_cast<const f32x2*>(p);
    x[0] = t[0];
    x[1] = t[1];
  } else {
    x[0] = *p;
  }
}
template <int R, int V>
__global__ __launch_bounds__(kCombWaveThreads) void combine_rows_kernel(CombArgs a, int64_t units) {
  const int D = a.d;
  const int spans = D / (64 * V);
  const int64_t unit = (int64_t)blockIdx.x * (kCombWaveThreads / 64) + (threadIdx.x >> 6);
  if (unit >= units) return;  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int64_t slot = unit / spans;
  const int pair = (int)(unit - slot * spans) * 64 * V + V * lane;
  const float* po = a.part_o + slot * a.nchunks * D + pair;
  const float* pml = a.part_ml + slot * a.nchunks * 2;
  float ov[R][V];
#pragma unroll
  for (int u = 0; u < R; ++u) load_v<V>(po + (int64_t)min(u, a.nchunks - 1) * D, ov[u]);
  const int cl = min(lane, a.nchunks - 1);
  const f32x2 ml = *reinterpret_cast<const f32x2*>(pml + 2 * cl);
  const int nch = a.nchunks;
  const bool live = lane < nch;
  const float M = wave_reduce<true>(live ? ml[0] : -INFINITY);
  const float wc = live && M != -INFINITY ? softmax_exp(ml[0] - M) : 0.f;
  const float L = wave_reduce<false>(live ? wc * ml[1] : 0.f);
  float acc[V];
#pragma unroll
  for (int e = 0; e < V; ++e) acc[e] = 0.f;
#pragma unroll
  for (int u = 0; u < R; ++u)
    if (u < nch) {
      const float wu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wc), u));
#pragma unroll
      for (int e = 0; e < V; ++e) acc[e] = fmaf(wu, ov[u][e], acc[e]);
    }
  float o[V];
#pragma unroll
  for (int e = 0; e < V; ++e) o[e] = L > 0.f ? acc[e] / L : 0.f;
  if (a.dh == D) {
    float* dst = a.o + slot * D + pair;
    if constexpr (V == 4) {
      *reinterpret_cast<f32x4*>(dst) = f32x4{o[0], o[1], o[2], o[3]};
    } else if constexpr (V == 2) {
      *reinterpret_cast<f32x2*>(dst) = f32x2{o[0], o[1]};
    } else {
      *dst = o[0];
    }
  } else {  // a padded launch: the stored head dim's outputs only
#pragma unroll
    for (int e = 0; e < V; ++e)
      if (pair + e < a.dh) a.o[slot * a.dh + pair + e] = o[e];
  }
}

__global__ void vexp_kernel(const float* x, float* y, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = softmax_exp(x[i]);
}

// The probabilities' exponential as the kernels take it: the natural-units
// argument scaled to base 2 (one fp32 rounding), then v_exp_f32.
__global__ void prob_exp_kernel(const float* x, float* y, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = exp2_hw(x[i] * kLog2e);
}

__global__ void zero_kernel(float* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

// ---------------------------------------------------------------------------
// Host side.

constexpr int kMaxChunk = 2048;
constexpr int kMaxSlots = 1 << 16;  // combine grid y: (sequence, head group) pairs per launch

// Process-wide settings (molot_hip_set_*): atomics, so a setter racing with
// launches on other host threads is well defined; a launch reads each once.
std::atomic<int> g_split_chunk{0};  // tokens per chunk, 0 = automatic
std::atomic<int> g_wgs_per_cu{0};   // workgroups per CU, 0 = the plan's own
std::atomic<int> g_dynamic{1};      // block order: 1 = claimed by waves as they free up, 0 = fixed
std::atomic<int> g_bf16_mfma{1};    // bf16 KV (D = 64, 128) on the matrix-core kernel
std::atomic<int> g_merge{-1};       // split-K merge: -1 automatic, 0 combine kernel, 1 in the launch

int knob(const std::atomic<int>& k) { return k.load(std::memory_order_relaxed); }

// Launch profiling (off by default): while on, every attention launch
// outside graph capture goes through hipExtLaunchKernelGGL with a start and
// a stop event per kernel, which HIP stamps from the dispatch itself (the
// kernel's execution, without the gap before it).  molot_hip_profile_end()
// waits for the events and returns the summed durations.
struct ProfRec {
  hipEvent_t a0, a1, c0, c1;  // attention kernel, combine kernel
  bool combine;
};
std::mutex g_prof_mu;
bool g_prof_on = false;
int g_prof_cap = 0;
std::vector<ProfRec> g_prof;

bool prof_active(void* stream) {
  if (!g_prof_on) return false;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing((hipStream_t)stream, &cap) != hipSuccess) return false;
  return cap == hipStreamCaptureStatusNone && (int)g_prof.size() < g_prof_cap;
}

hipEvent_t prof_event() {
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

void prof_destroy(ProfRec& r) {
  for (hipEvent_t e : {r.a0, r.a1, r.c0, r.c1})
    if (e) (void)hipEventDestroy(e);
}

struct WsKey {
  int dev;
  void* stream;
  bool operator<(const WsKey& o) const {
    return dev != o.dev ? dev < o.dev : stream < o.stream;
  }
};
// Per-(device, stream) workspace of the split-K partials, grown on demand.
// Layout: [u64 ctr[kMaxSlots] | partials].  The arrival words of the
// in-launch merge are zeroed once, when the buffer is allocated (a fill
// kernel on the stream, ordered before any launch that uses them), and
// every launch leaves them at zero.  The partials are filled and read
// within a step (by the attention kernel, or by it and the combine kernel
// next on the same stream), so they need no clearing and hold nothing
// between steps.  An outgrown buffer is retired, never freed: a graph
// captured earlier on the stream still points at it (workspaces are small).
constexpr size_t kCtrBytes = sizeof(unsigned long long) * (size_t)kMaxSlots;
struct WsBuf {
  void* ptr = nullptr;
  size_t bytes = 0;  // partials
};
std::mutex g_ws_mu;
std::map<WsKey, WsBuf> g_ws;
std::vector<void*> g_retired;

__global__ void zero_kernel(float* p, int64_t n);
bool xcd_map_ok(int dev);

int workspace(void* stream, size_t bytes, unsigned long long** ctr, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  std::lock_guard<std::mutex> lk(g_ws_mu);
  WsBuf& w = g_ws[WsKey{dev, stream}];
  if (!w.ptr || w.bytes < bytes) {
    // a graph being captured cannot allocate: the caller sizes the
    // workspace with one launch of the shape before capturing
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing((hipStream_t)stream, &cap);
    if (e != hipSuccess) return (int)e;
    if (cap != hipStreamCaptureStatusNone) return MOLOT_ENOWS;
    (void)xcd_map_ok(dev);  // the one-time dispatch check, outside any capture
    if (w.ptr) g_retired.push_back(w.ptr);
    w = WsBuf{};
    const size_t want = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
    void* p = nullptr;
    e = hipMalloc(&p, kCtrBytes + want);
    if (e != hipSuccess) return (int)e;
    hipLaunchKernelGGL(zero_kernel, dim3((unsigned)(kCtrBytes / 4 / 256)), dim3(256), 0,
                       (hipStream_t)stream, reinterpret_cast<float*>(p), (int64_t)(kCtrBytes / 4));
    e = hipGetLastError();
    if (e != hipSuccess) {
      (void)hipFree(p);
      return (int)e;
    }
    w.ptr = p;
    w.bytes = want;
  }
  *ctr = reinterpret_cast<unsigned long long*>(w.ptr);
  *out = reinterpret_cast<char*>(w.ptr) + kCtrBytes;
  return 0;
}

// Per-(device, stream) workspace of the prefill's pre-split K/V pieces,
// grown to at least twice its last size (so the retired buffers, which a
// captured graph may still point at, total less than the live one).  Under
// stream capture it cannot grow: the caller then splits per tile instead.
std::map<WsKey, WsBuf> g_pieces_ws;
constexpr size_t kMaxPiecesBytes = (size_t)1 << 30;  // the prefill's pre-split workspace

int pieces_workspace(void* stream, size_t bytes, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  std::lock_guard<std::mutex> lk(g_ws_mu);
  WsBuf& w = g_pieces_ws[WsKey{dev, stream}];
  if (!w.ptr || w.bytes < bytes) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing((hipStream_t)stream, &cap);
    if (e != hipSuccess) return (int)e;
    if (cap != hipStreamCaptureStatusNone) return MOLOT_ENOWS;
    // at most kMaxPiecesBytes (bytes never exceeds it), so the live buffer
    // and the retired ones a captured graph may still hold stay under 2 GiB
    const size_t want = std::min(std::max(bytes, 2 * w.bytes), std::max(bytes, kMaxPiecesBytes));
    void* p = nullptr;
    e = hipMalloc(&p, want);
    if (e != hipSuccess) return (int)e;
    if (w.ptr) g_retired.push_back(w.ptr);
    w.ptr = p;
    w.bytes = want;
  }
  *out = w.ptr;
  return 0;
}

// Dispatch check for the in-launch merge, once per device: a probe launch
// records the XCD (hardware register XCC_ID) of every workgroup of a 4096-
// workgroup grid, and the merge is used only if workgroup i always ran on
// the same XCD as workgroup i % 8 (MI355X's round-robin dispatch in its
// single-partition mode; with one XCD per device the check holds
// trivially).  Read-only after the first call for a device.
__device__ int g_xcc_probe[4096];
__global__ void xcc_probe_kernel() {
  if (threadIdx.x == 0)
    g_xcc_probe[blockIdx.x] = xcc_id();
}
std::mutex g_xcd_mu;
std::map<int, bool> g_xcd_ok;

bool xcd_map_ok(int dev) {
  std::lock_guard<std::mutex> lk(g_xcd_mu);
  auto it = g_xcd_ok.find(dev);
  if (it != g_xcd_ok.end()) return it->second;
  bool ok = false;
  std::vector<int> xcc(4096, -1);
  hipStream_t st = nullptr;
  if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) == hipSuccess) {
    hipLaunchKernelGGL(xcc_probe_kernel, dim3(4096), dim3(64), 0, st);
    if (hipGetLastError() == hipSuccess &&
        hipMemcpyFromSymbolAsync(xcc.data(), HIP_SYMBOL(g_xcc_probe), sizeof(int) * 4096, 0,
                                 hipMemcpyDeviceToHost, st) == hipSuccess &&
        hipStreamSynchronize(st) == hipSuccess) {
      ok = true;
      for (int i = 0; i < 4096; ++i) ok = ok && xcc[i] >= 0 && xcc[i] == xcc[i % 8];
    }
    (void)hipStreamDestroy(st);
  }
  g_xcd_ok[dev] = ok;
  return ok;
}

bool xcd_ok_cached(int dev) {
  std::lock_guard<std::mutex> lk(g_xcd_mu);
  auto it = g_xcd_ok.find(dev);
  return it != g_xcd_ok.end() && it->second;
}

// Scratch of the no-allocation entry point (molot_hip_decode_step_noalloc):
// the split-K partials of one launch, in device memory that exists from
// module load to process end on every device the library runs on.  Host
// code never passes `scratch` itself (on the host it is only a stand-in
// for the symbol): noalloc_scratch() resolves the device's address once per
// device with hipGetSymbolAddress and hands out that pointer.  Every call
// on a device shares its array; the partials are written and read within
// one step, so nothing needs clearing between calls, and calls that
// overlap on one device race on it.
constexpr size_t kScratchBytes = (size_t)4 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
std::mutex g_scratch_mu;
std::map<int, void*> g_scratch_ptr;

int noalloc_scratch(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  auto it = g_scratch_ptr.find(dev);
  if (it == g_scratch_ptr.end()) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));  // this device is current
    if (e != hipSuccess) return (int)e;
    if (!ptr) return (int)hipErrorInvalidSymbol;
    it = g_scratch_ptr.emplace(dev, ptr).first;
  }
  *out = it->second;
  return 0;
}

int g_num_cus = 0;
int num_cus() {
  if (g_num_cus) return g_num_cus;
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess &&
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
      cus > 0)
    g_num_cus = cus;
  else
    cus = 256;
  return cus;
}

int pick_gh(int G) {
  if (G % 8 == 0) return 8;
  if (G % 4 == 0) return 4;
  if (G % 2 == 0) return 2;
  return 1;
}

// Tokens per chunk: enough chunks that the launch holds `wpc` workgroups
// per CU (one by default: a workgroup fills its CU), rounded up to a
// multiple of `align` rows (a forced size too: the matrix-core kernel deals
// 32-row tiles to the chunks, and every chunk must get one).
int plan_chunk(int span, int rows_of_wgs, int align, int wpc, int split, int wpcu) {
  int chunk = split;
  if (chunk <= 0) {
    const long target = (long)(wpcu > 0 ? wpcu : wpc) * num_cus();
    long nch = (target + rows_of_wgs - 1) / rows_of_wgs;
    if (nch < 1) nch = 1;
    chunk = (int)((span + nch - 1) / nch);
  }
  chunk = (chunk + align - 1) / align * align;
  if (chunk > kMaxChunk) chunk = kMaxChunk;
  if (chunk < 8) chunk = 8;
  return chunk;
}

// Chunking + workspace of one launch.  `span` bounds every sequence's row
// range tiled by chunks (cache rows only when the kernel folds in the new
// token); B * nkv * subgroups slots share each chunk index.  `cyclic`: the
// kernel deals `align`-row tiles to the chunks round robin (the matrix-core
// kernel on a contiguous cache), so only the chunk count matters: the
// workgroup target's, at most one chunk per tile (a.chunk is then nominal).
//
// A split context is merged in the launch itself (arrive_and_merge) when the
// device dispatches workgroup i to XCD i % 8 and every chunk of a slot can
// run on one XCD: with the grid's slot index fastest that holds when the
// slot count is a multiple of 8; fewer than 8 slots take a 1-D grid that
// puts slot s on XCD s (xmap).  Other slot counts, token-major Q8 launches
// (whose grid groups the heads of a chunk on one XCD instead) and slots of
// more than kMergeMaxChunks chunks use combine_kernel.
int plan_launch(AttnArgs& a, int d, int span, int gh, int nsubs, int B, int align, int wpc,
                void* stream, bool cyclic = false) {
  const int rows = a.nkv * nsubs * B;
  const int split = knob(g_split_chunk), wpcu = knob(g_wgs_per_cu);
  if (cyclic) {
    const long tiles = span > 0 ? ((long)span + align - 1) / align : 1;
    long nch;
    if (split > 0) {
      const long ch = ((long)split + align - 1) / align * align;
      nch = span > 0 ? (span + ch - 1) / ch : 1;
    } else {
      const long target = (long)(wpcu > 0 ? wpcu : wpc) * num_cus();
      nch = (target + rows - 1) / rows;
    }
    nch = std::max(1L, std::min({nch, tiles, (long)kMaxChunks}));
    a.nchunks = (int)nch;
    a.chunk = (int)((tiles + nch - 1) / nch * align);
  } else {
    a.chunk = plan_chunk(span > 0 ? span : 1, rows, align, wpc, split, wpcu);
    a.nchunks = span > 0 ? (span + a.chunk - 1) / a.chunk : 1;
    // bound the chunk count (grid x, and the combine's per-pair loop)
    while (a.nchunks > kMaxChunks && a.chunk < kMaxChunk) {
      a.chunk *= 2;
      a.nchunks = (span + a.chunk - 1) / a.chunk;
    }
    if (a.nchunks > kMaxChunks) return MOLOT_ENOTSUP;
  }
  a.part_o = nullptr;
  a.part_ml = nullptr;
  a.qrot = nullptr;
  a.ctr = nullptr;
  a.xmap = 0;
  a.slots = rows;
  a.mrg = 0;
  if (a.nchunks == 1) return 0;  // single chunk: written directly, no combine
  if ((long)rows > kMaxSlots) return MOLOT_ENOTSUP;
  const size_t P = (size_t)gh * d;
  const size_t po = (size_t)rows * a.nchunks * P;
  const size_t pml = (size_t)rows * a.nchunks * gh * 2;
  const size_t qr = (size_t)rows * P;
  void* ws = nullptr;
  unsigned long long* ctr = nullptr;
  const size_t need = sizeof(float) * (po + pml + qr);
  if (a.ext_ws) {
    // a caller-provided workspace (molot_hip_decode_step_noalloc): no
    // allocation, and the combine kernel merges (no counters to keep)
    if ((int64_t)need > a.ext_ws_bytes) return MOLOT_E2BIG;
    a.part_o = reinterpret_cast<float*>(a.ext_ws);
    a.part_ml = a.part_o + po;
    a.qrot = a.part_ml + pml;
    return 0;
  }
  const int st = workspace(stream, need, &ctr, &ws);
  if (st) return st;
  a.part_o = reinterpret_cast<float*>(ws);
  a.part_ml = a.part_o + po;
  a.qrot = a.part_ml + pml;
  int dev = 0;
  // automatic: in the launch when the slots fill the 8 XCDs evenly on a
  // contiguous cache and the context is long (measured, 32q/8kv/d128 fp32:
  // step 27.3 -> 26.4 us at n = 16385; at n = 4097 the combine kernel is
  // 0.1 us faster; fewer slots would leave XCDs idle under the 1-D map, and
  // batches of short paged sequences merge few chunks cheaply in the
  // combine kernel: c4 234.8 against 239.3 us).  The matrix-core kernel
  // keeps the combine kernel (launch_mfma).
  const int mk = knob(g_merge);
  const bool want =
      mk > 0 || (mk < 0 && rows % 8 == 0 && !a.block_table && span >= kMergeAutoSpan);
  const bool merge = want && !a.chunk_fast && (rows % 8 == 0 || rows < 8) &&
                     a.nchunks <= kMergeMaxChunks && hipGetDevice(&dev) == hipSuccess &&
                     xcd_ok_cached(dev);
  if (merge) {
    a.ctr = ctr;
    a.xmap = rows % 8 != 0;
    a.mrg = merge_lds_floats(gh);
  }
  return 0;
}

// The combine kernel merges this launch's chunks instead.
void no_merge(AttnArgs& a) {
  a.ctr = nullptr;
  a.xmap = 0;
  a.mrg = 0;
}

using AttnFn = void (*)(AttnArgs);

// geometry of this thread's last attention launch (molot_hip_last_plan)
thread_local int t_last_nchunks = 0;
thread_local int t_last_chunk = 0;

// Dynamic LDS a workgroup may take (the CU's 160 KiB).
constexpr size_t kMaxLds = 160 * 1024;

// Launches an attention kernel of a planned problem and, for a split
// context, combine_kernel after it on the same stream.
int launch_pair(AttnFn kern, int threads, size_t lds, AttnArgs a, int gh, int d, int nsubs,
                int B, bool paged, bool rope, void* stream) {
  if (lds > kMaxLds) return (int)hipErrorInvalidConfiguration;
  if ((gh * d) % kCombPairs || d % kCombPairs) return MOLOT_ENOTSUP;  // combine tiling
  t_last_nchunks = a.nchunks;
  t_last_chunk = a.chunk;
  a.dynamic = knob(g_dynamic);
  std::lock_guard<std::mutex> plk(g_prof_mu);
  const bool prof = !a.ext_ws && prof_active(stream);
  const bool combine = a.nchunks > 1 && !a.ctr;  // a second launch merges the chunks
  ProfRec pr{nullptr, nullptr, nullptr, nullptr, combine};
  // Workgroup i runs on XCD i % 8 (its L2 and its share of the CUs), and
  // workgroups are dispatched in linear order.  With the (KV head, subgroup)
  // index fastest, every XCD gets the same heads' share of every chunk and
  // sequence (equal work however the chunks of a batch differ in length),
  // and the chunk index slowest makes the XCDs stream the same rows at the
  // same time.  chunk_fast (Q8 caches) groups by chunk instead: the KV heads
  // of one token share 128-byte lines (token-major: head rows of d bytes at
  // t*R + h*d, the token's scales after them; paged: the page's scales
  // after its codes, 64 bytes a head), so all heads of a (sequence, chunk)
  // pair go to one XCD, whose L2 then fetches each shared line once.  A 1-D
  // grid of 8 * ceil(pairs / 8) * heads workgroups: id runs pair
  // (id / 8 / heads) * 8 + id % 8 (chunk slot pair / B of sequence pair % B)
  // and head (id / 8) % heads, so each pair is on one XCD whatever the
  // counts, its heads are dispatched together, and the padding ids exit at
  // once.
  // xmap (in-launch merge, fewer than 8 slots): a 1-D grid of 8 * nchunks
  // workgroups, id running chunk slot id / 8 of slot id % 8, so each slot's
  // chunks share an XCD; ids of absent slots exit at once.
  const dim3 grid = a.chunk_fast
                        ? dim3((unsigned)(((int64_t)B * a.nchunks + 7) / 8 * 8 * a.nkv * nsubs), 1, 1)
                        : a.xmap ? dim3((unsigned)(8 * a.nchunks), 1, 1)
                                 : dim3(a.nkv * nsubs, B, a.nchunks);
  if (prof) {
    pr.a0 = prof_event();
    pr.a1 = prof_event();
    hipExtLaunchKernelGGL(kern, grid, dim3(threads), lds, (hipStream_t)stream, pr.a0, pr.a1, 0,
                          a);
  } else {
    hipLaunchKernelGGL(kern, grid, dim3(threads), lds, (hipStream_t)stream, a);
  }
  int st = (int)hipGetLastError();
  if (st || !combine) {
    if (prof) g_prof.push_back(pr);
    return st;
  }
  CombArgs cb{};
  cb.part_o = a.part_o;
  cb.part_ml = a.part_ml;
  cb.qrot = a.qrot;
  cb.o = a.o;
  cb.q_out = a.q_out;
  cb.seq_lens = a.seq_lens;
  cb.pos_arr = a.pos_arr;
  cb.nq = a.nq;
  cb.nkv = a.nkv;
  cb.gh = gh;
  cb.nsub = nsubs;
  cb.d = d;
  cb.dh = a.dh;
  cb.nchunks = a.nchunks;
  cb.chunk = a.chunk;
  cb.window = a.window;
  cb.rope = rope ? 1 : 0;
  cb.paged = paged ? 1 : 0;
  cb.fold = rope && a.fold ? 1 : 0;
  cb.pf = rope ? 0 : a.pf;
  cb.pos0 = a.pos;
  cb.n = a.n;
  // At most 8 chunks (batches of sequences: many slots, few chunks): one
  // wave per 64 pairs (combine_wave_kernel<R>, R = 4 or 8 o loads per lane).
  // More chunks: combine_kernel, whose 4 phases per pair keep the loads per
  // lane at 8 a round (the wave kernel issued 32-64 per lane and was 0.4 us
  // slower at 32 and 64 chunks).
  const int P = gh * d;
  const int wthreads = P % 256 == 0 ? 256 : (P % 128 == 0 ? 128 : 64);
  const int slots = a.nkv * nsubs * B;
  using CombFn = void (*)(CombArgs);
  const bool wave = a.nchunks <= 8;
  const CombFn ck = a.nchunks <= 4 ? combine_wave_kernel<4>
                    : wave         ? combine_wave_kernel<8>
                                   : combine_kernel;
  cb.pairs = comb_pairs(a.nchunks);
  const dim3 cgrid = wave ? dim3(slots, P / wthreads) : dim3(slots, P / cb.pairs);
  const dim3 cblock = wave ? dim3(wthreads) : dim3(kCombThreads);
  const size_t clds = wave ? 0 : sizeof(float) * (size_t)comb_lds_floats(a.nchunks);  // <= 33 KB
  if (prof) {
    pr.c0 = prof_event();
    pr.c1 = prof_event();
    hipExtLaunchKernelGGL(ck, cgrid, cblock, clds, (hipStream_t)stream, pr.c0, pr.c1, 0, cb);
    g_prof.push_back(pr);
  } else {
    hipLaunchKernelGGL(ck, cgrid, cblock, clds, (hipStream_t)stream, cb);
  }
  return (int)hipGetLastError();
}

// A planned launch of attn_kernel with configuration C.
template <int D, int GH, typename T, bool PAGED, bool ROPE, bool PAD, typename C>
int launch_planned(AttnArgs a, int nsubs, int B, void* stream) {
  if (a.mrg && sizeof(float) * (size_t)Lds(D, GH, C::NW, C::RB, a.chunk, a.page_shift, PAGED,
                                           a.mrg).total > kMaxLds)
    no_merge(a);  // the merge's statistics do not fit beside the kernel's LDS
  const Lds L(D, GH, C::NW, C::RB, a.chunk, a.page_shift, PAGED, a.mrg);
  return launch_pair(attn_kernel<D, GH, T, PAGED, ROPE, PAD, C>, C::NT, sizeof(float) * (size_t)L.total,
                     a, GH, D, nsubs, B, PAGED, ROPE, stream);
}

template <int D, int GH, typename T, bool PAGED, bool ROPE, bool PAD, typename C>
int launch_cfg(AttnArgs a, int span, int nsubs, int B, void* stream) {
  // Q8 (d = 256): the heads of a token share 128-byte lines (see launch_pair)
  a.chunk_fast = sizeof(T) == 1;
  a.nseq = B;
  // contiguous caches: 32-row groups dealt round robin (the kernel's gmap);
  // prefill rows, like paged batches, tile each row's range in contiguous
  // chunks and merge them in the combine kernel
  const bool perseq = PAGED || (!ROPE && a.pf);
  int st = plan_launch(a, D, span, GH, nsubs, B, perseq ? C::RB : 32, 1, stream, !perseq);
  if (st) return st;
  if (a.pf) no_merge(a);
  if constexpr (sizeof(T) == 1 && C::NW > 8) {
    // Q8 chunks of at most 4 blocks a wave on 8 waves: a 1024-token window
    // of 8q/4kv/d256 (32-row chunks) 14.45 -> 10.9 us per step; 512-row
    // chunks (32k tokens, no window) stay on 16 waves (26.0 against 27.8 us)
    if (a.chunk <= 8 * 4 * C::RB)
      return launch_planned<D, GH, T, PAGED, ROPE, PAD,
                            Cfg<D, GH, T, C::LPR, C::RB, 8, C::NBUF>>(a, nsubs, B, stream);
  }
  return launch_planned<D, GH, T, PAGED, ROPE, PAD, C>(a, nsubs, B, stream);
}

// bf16 or Q8 KV, D = 64 or 128: the matrix-core kernel.  Workgroups per CU
// in the plan (measured): a contiguous cache 1 (c5 kernel 96.0 -> 93.2 us
// against 2; with two per CU the one dispatched second streams at about
// half the rate of the first, and the chunks left to it form the tail);
// paged batches are cut finer, their sequences differing in length: bf16
// 16 (c4 240.2 -> 235.6 us against 8), Q8 8 (c4q8: 141.5 us, 150.1 at 16).
template <int D, int GH, bool PAGED, bool ROPE, bool Q8>
int launch_mfma(AttnArgs a, int span, int nsubs, int B, void* stream) {
  constexpr int kWpc = PAGED ? (Q8 ? 8 : 16) : 1;
  a.chunk_fast = Q8;
  a.nseq = B;
  int st = plan_launch(a, D, span, GH, nsubs, B, kTile, kWpc, stream, !PAGED);
  if (st) return st;
  // by default the combine kernel: its four waves per workgroup would fold
  // the chunks in sequential rounds (c5: 111.7 against 99.5 us per step)
  if (knob(g_merge) < 0) no_merge(a);
  if (a.mrg && sizeof(float) * (size_t)LdsM(D, GH, a.chunk, a.page_shift, PAGED, Q8, a.mrg).total >
                   kMaxLds)
    no_merge(a);
  const LdsM L(D, GH, a.chunk, a.page_shift, PAGED, Q8, a.mrg);
  return launch_pair(attn_mfma_kernel<D, GH, PAGED, ROPE, Q8>, kMfmaThreads,
                     sizeof(float) * (size_t)L.total, a, GH, D, nsubs, B, PAGED, ROPE, stream);
}

template <int D, int GH, typename T, bool PAGED, bool ROPE, bool PAD>
int launch_attn(const AttnArgs& a, int span, int nsubs, int B, void* stream) {
  return launch_cfg<D, GH, T, PAGED, ROPE, PAD, typename Tune<D, GH, T>::C>(a, span, nsubs, B,
                                                                           stream);
}

// Query heads per workgroup: up to 8 (d <= 256) or 4 (d = 512, whose
// 8-head workgroup would need 99 KB of LDS for its waves' partial o; 8 q
// heads of a KV head then run as two subgroups reading the rows twice).
constexpr int kMaxGhWide = 4;
template <int D, typename T, bool PAGED, bool ROPE, bool PAD>
int dispatch_gh(int gh, const AttnArgs& a, int span, int nsubs, int B, void* st) {
  switch (gh) {
    case 1: return launch_attn<D, 1, T, PAGED, ROPE, PAD>(a, span, nsubs, B, st);
    case 2: return launch_attn<D, 2, T, PAGED, ROPE, PAD>(a, span, nsubs, B, st);
    case 4: return launch_attn<D, 4, T, PAGED, ROPE, PAD>(a, span, nsubs, B, st);
    case 8:
      if constexpr (D <= 256 && !(sizeof(T) == 1 && D <= 128))
        return launch_attn<D, 8, T, PAGED, ROPE, PAD>(a, span, nsubs, B, st);
      break;
  }
  return MOLOT_EINVAL;
}

// The vector-ALU kernels are built for D = 64, 128, 256 and 512; any other
// even head dim d <= 512 runs padded in the next of them (q zero-padded to
// D, K/V rows read at their stored length d).
template <int D, typename T, bool PAGED, bool ROPE>
int dispatch_pad(int d, int gh, const AttnArgs& a, int span, int nsubs, int B, void* st) {
  return d == D ? dispatch_gh<D, T, PAGED, ROPE, false>(gh, a, span, nsubs, B, st)
                : dispatch_gh<D, T, PAGED, ROPE, true>(gh, a, span, nsubs, B, st);
}

template <typename T, bool PAGED, bool ROPE>
int dispatch_d(int d, int gh, const AttnArgs& a, int span, int nsubs, int B, void* st) {
  if constexpr (sizeof(T) == 1) {  // Q8: 64 and 128 whole take the matrix cores (run_attn)
    if (d < 64) return dispatch_gh<64, T, PAGED, ROPE, true>(gh, a, span, nsubs, B, st);
    if (d < 128) return dispatch_gh<128, T, PAGED, ROPE, true>(gh, a, span, nsubs, B, st);
  } else {
    if (d <= 64) return dispatch_pad<64, T, PAGED, ROPE>(d, gh, a, span, nsubs, B, st);
    if (d <= 128) return dispatch_pad<128, T, PAGED, ROPE>(d, gh, a, span, nsubs, B, st);
  }
  if (d <= 256) return dispatch_pad<256, T, PAGED, ROPE>(d, gh, a, span, nsubs, B, st);
  return dispatch_pad<512, T, PAGED, ROPE>(d, gh, a, span, nsubs, B, st);
}

template <bool PAGED, bool ROPE>
int dispatch_attn(int d, int kv_dtype, int gh, const AttnArgs& a, int span, int nsubs, int B,
                  void* st) {
  if (kv_dtype == MOLOT_KV_F32) return dispatch_d<float, PAGED, ROPE>(d, gh, a, span, nsubs, B, st);
  if (kv_dtype == MOLOT_KV_Q8)  // 64 and 128 take the matrix cores (run_attn)
    return dispatch_d<q8_t, PAGED, ROPE>(d, gh, a, span, nsubs, B, st);
  return dispatch_d<bf16_t, PAGED, ROPE>(d, gh, a, span, nsubs, B, st);
}

// Head dims the prefill's matrix-core kernel is built for; decode on fp32
// and bf16 caches takes any even d up to 512, Q8 caches q8_d: any multiple
// of 4 (a token's fp32 scales follow its nkv*d codes, 4-byte aligned).
bool supported_d(int d) { return d == 64 || d == 128 || d == 256; }
bool decode_d(int d) { return d >= 2 && d <= 512 && d % 2 == 0; }
bool q8_d(int d) { return d >= 4 && d <= 512 && d % 4 == 0; }

bool valid_kv(int kv_dtype) {
  return kv_dtype == MOLOT_KV_F32 || kv_dtype == MOLOT_KV_BF16 || kv_dtype == MOLOT_KV_Q8;
}

// bytes of one K/V element (Q8: one code)
int kv_esz(int kv_dtype) { return kv_dtype == MOLOT_KV_F32 ? 4 : kv_dtype == MOLOT_KV_BF16 ? 2 : 1; }

// Q8 byte layouts: a token-major row (codes, then the nkv scales padded to
// 16 bytes) and a paged block (codes [nkv][page][d], then scales [nkv][page])
int64_t q8_row_bytes(int nkv, int d) { return (int64_t)nkv * d + ((4 * (int64_t)nkv + 15) & ~15); }
int64_t q8_block_bytes(int nkv, int d, int page) { return (int64_t)nkv * page * (d + 4); }

int check_common(int nq, int nkv, int d, int kv_dtype) {
  if (nq <= 0 || nkv <= 0 || nq % nkv != 0) return MOLOT_EINVAL;
  if (!valid_kv(kv_dtype)) return MOLOT_EINVAL;
  if (!decode_d(d)) return MOLOT_ENOTSUP;
  if (kv_dtype == MOLOT_KV_Q8 && !q8_d(d)) return MOLOT_ENOTSUP;  // Q8: 64, 128, 256, 512
  return 0;
}

// The strides and scale offsets of the token-major cache [cap][nkv*d]
// (Q8: its byte layout) in a or r.
template <typename A>
void token_major(A& a, int nkv, int d, int kv_dtype) {
  const bool q8 = kv_dtype == MOLOT_KV_Q8;
  a.tok_stride = q8 ? q8_row_bytes(nkv, d) : (int64_t)nkv * d;
  a.head_stride = d;
  a.sc_off = (int64_t)nkv * d;
  a.sc_head = 4;
}

// The same for pages [block][nkv][page][d].
template <typename A>
void paged_layout(A& a, int nkv, int d, int page, int kv_dtype) {
  a.tok_stride = d;
  a.head_stride = (int64_t)page * d;
  a.block_stride =
      kv_dtype == MOLOT_KV_Q8 ? q8_block_bytes(nkv, d, page) : (int64_t)nkv * page * d;
  a.sc_off = (int64_t)nkv * page * d;
  a.sc_head = 4LL * page;
}

// Q8 pages: 16-byte aligned blocks need nkv*page scales to fill 16 bytes
bool q8_pages_ok(int nkv, int page, int kv_dtype) {
  return kv_dtype != MOLOT_KV_Q8 || ((int64_t)nkv * page) % 4 == 0;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int zero_out(float* O, int64_t count, hipStream_t st) {
  if (count <= 0) return 0;
  const int64_t blocks = (count + 255) / 256;
  hipLaunchKernelGGL(zero_kernel, dim3((unsigned)blocks), dim3(256), 0, st, O, count);
  return (int)hipGetLastError();
}

template <int D, bool PAGED, bool ROPE, bool Q8>
int dispatch_mfma(int gh, const AttnArgs& a, int span, int nsubs, int B, void* st) {
  switch (gh) {
    case 1: return launch_mfma<D, 1, PAGED, ROPE, Q8>(a, span, nsubs, B, st);
    case 2: return launch_mfma<D, 2, PAGED, ROPE, Q8>(a, span, nsubs, B, st);
    case 4: return launch_mfma<D, 4, PAGED, ROPE, Q8>(a, span, nsubs, B, st);
    case 8: return launch_mfma<D, 8, PAGED, ROPE, Q8>(a, span, nsubs, B, st);
    case 16: return launch_mfma<D, 16, PAGED, ROPE, Q8>(a, span, nsubs, B, st);
  }
  return MOLOT_EINVAL;
}

template <bool PAGED, bool ROPE>
int run_attn(AttnArgs& a, int d, int kv_dtype, int span, int B, void* stream) {
  a.dh = d;
  const int G = a.nq / a.nkv;
  const bool q8 = kv_dtype == MOLOT_KV_Q8;
  if ((q8 || (kv_dtype == MOLOT_KV_BF16 && g_bf16_mfma)) && (d == 64 || d == 128)) {
    // up to 16 q heads of a group share each K/V tile on the MFMA columns;
    // Q8 caches of D = 64, 128 run here, D = 256 and 512 on the vector-ALU
    // kernel
    const int gh = G % 16 == 0 ? 16 : pick_gh(G);
    const int nsubs = G / gh;
    if (q8)
      return d == 64 ? dispatch_mfma<64, PAGED, ROPE, true>(gh, a, span, nsubs, B, stream)
                     : dispatch_mfma<128, PAGED, ROPE, true>(gh, a, span, nsubs, B, stream);
    return d == 64 ? dispatch_mfma<64, PAGED, ROPE, false>(gh, a, span, nsubs, B, stream)
                   : dispatch_mfma<128, PAGED, ROPE, false>(gh, a, span, nsubs, B, stream);
  }
  // Q8 rows padded to D <= 128 hold 16 q elements a lane per head: at most
  // 4 heads a workgroup there too
  const int gh = d > 256 || (q8 && d < 128) ? std::min(pick_gh(G), kMaxGhWide) : pick_gh(G);
  const int nsubs = G / gh;
  return dispatch_attn<PAGED, ROPE>(d, kv_dtype, gh, a, span, nsubs, B, stream);
}

// The layer's norms of the fresh q, k and v (forward.h:554, 562-563).
struct Norms {
  const float* q = nullptr;  // per-head q weights [d], NULL: none
  const float* k = nullptr;  // per-head k weights [d], NULL: none
  int v = 0;                 // v over all nkv*d values, no weights
  float eps = 0.f;
};

bool norms_ok(const Norms& nm) { return nm.eps >= 0.f && nm.eps < INFINITY; }

using PfFn = void (*)(PfArgs);
std::atomic<int> g_presplit{1};  // molot_hip_set_prefill_presplit

template <int D, typename T, bool PAGED>
PfFn pf_kernel_w(int pw) {
  if (pw == 8) return prefill_mfma16_kernel<D, T, PAGED, 8>;
  return prefill_mfma16_kernel<D, T, PAGED, 4>;
}

template <typename T, bool PAGED>
PfFn pf_kernel_d(int d, int pw) {
  if (d == 64) return pf_kernel_w<64, T, PAGED>(pw);
  if (d == 128) return pf_kernel_w<128, T, PAGED>(pw);
  if constexpr (!std::is_same<T, q8_t>::value) return pf_kernel_w<256, T, PAGED>(pw);
  return nullptr;  // Q8 prefill: d = 64, 128
}

// The prefill kernel over pre-split pieces (any cache type but bf16).
PfFn pf_kernel_pre(int d, int pw) {
  if (d == 64) return pw == 8 ? prefill_mfma16_kernel<64, float, false, 8, true>
                              : prefill_mfma16_kernel<64, float, false, 4, true>;
  if (d == 128) return pw == 8 ? prefill_mfma16_kernel<128, float, false, 8, true>
                               : prefill_mfma16_kernel<128, float, false, 4, true>;
  return pw == 8 ? prefill_mfma16_kernel<256, float, false, 8, true>
                 : prefill_mfma16_kernel<256, float, false, 4, true>;
}

using SplitFn = void (*)(PfArgs, uint16_t*);
SplitFn pf_split(int d, int kv_dtype, bool paged) {
  if (kv_dtype == MOLOT_KV_Q8) {
    if (d == 64) return paged ? pf_split_kernel<64, q8_t, true> : pf_split_kernel<64, q8_t, false>;
    if (d == 128)
      return paged ? pf_split_kernel<128, q8_t, true> : pf_split_kernel<128, q8_t, false>;
    return paged ? pf_split_kernel<256, q8_t, true> : pf_split_kernel<256, q8_t, false>;
  }
  if (d == 64) return paged ? pf_split_kernel<64, float, true> : pf_split_kernel<64, float, false>;
  if (d == 128) return paged ? pf_split_kernel<128, float, true> : pf_split_kernel<128, float, false>;
  return paged ? pf_split_kernel<256, float, true> : pf_split_kernel<256, float, false>;
}

// The prefill kernel of a head dim (64, 128, 256), cache type, layout and
// wave count (pw: 4, or 8 where the instance has it).
PfFn pf_kernel(int d, int kv_dtype, bool paged, int pw) {
  if (kv_dtype == MOLOT_KV_Q8)
    return paged ? pf_kernel_d<q8_t, true>(d, pw) : pf_kernel_d<q8_t, false>(d, pw);
  if (kv_dtype == MOLOT_KV_F32)
    return paged ? pf_kernel_d<float, true>(d, pw) : pf_kernel_d<float, false>(d, pw);
  return paged ? pf_kernel_d<bf16_t, true>(d, pw) : pf_kernel_d<bf16_t, false>(d, pw);
}

}  // namespace

// ===========================================================================
// C ABI
extern "C" {

const char* molot_hip_strerror(int status) {
  switch (status) {
    case MOLOT_OK: return "ok";
    case MOLOT_EINVAL: return "molot_amd: invalid argument";
    case MOLOT_ENOTSUP:
      return "molot_amd: unsupported shape (an even head dim up to 512; Q8 caches a multiple "
             "of 4 up to 512)";
    case MOLOT_ENOSPC: return "molot_amd: KV cache full";
    case MOLOT_ENOWS:
      return "molot_amd: workspace not sized for this shape on a capturing stream (launch the "
             "shape once before capturing)";
    case MOLOT_E2BIG:
      return "molot_amd: the split-K partials of this shape exceed the 4 MiB scratch of "
             "molot_hip_decode_step_noalloc";
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "molot_amd: unknown status";
}

const char* molot_hip_version(void) { return "molot_amd 0.2"; }

int molot_hip_q8_row_bytes(int nkv, int d) {
  return nkv > 0 && d > 0 ? (int)q8_row_bytes(nkv, d) : 0;
}

int64_t molot_hip_q8_block_bytes(int nkv, int d, int page) {
  return nkv > 0 && d > 0 && page > 0 ? q8_block_bytes(nkv, d, page) : 0;
}

void molot_rope_inv_freq(float base, int d, float* out) {
  for (int i = 0; i < d / 2; ++i) out[i] = 1.0f / powf(base, (2.0f * (float)i) / (float)d);
}

void molot_hip_set_split_chunk(int tokens) { g_split_chunk = tokens > 0 ? tokens : 0; }

int molot_hip_last_plan(int* nchunks, int* chunk) {
  if (!nchunks || !chunk || t_last_nchunks <= 0) return MOLOT_EINVAL;
  *nchunks = t_last_nchunks;
  *chunk = t_last_chunk;
  return 0;
}

void molot_hip_set_block_order(int dynamic) { g_dynamic = dynamic ? 1 : 0; }

void molot_hip_set_bf16_path(int mfma) { g_bf16_mfma = mfma ? 1 : 0; }

int molot_hip_profile_begin(int max_launches) {
  if (max_launches <= 0) return MOLOT_EINVAL;
  std::lock_guard<std::mutex> lk(g_prof_mu);
  for (ProfRec& r : g_prof) prof_destroy(r);
  g_prof.clear();
  g_prof.reserve(max_launches);
  g_prof_cap = max_launches;
  g_prof_on = true;
  return 0;
}

int molot_hip_profile_end(float* attn_ms, float* combine_ms, int* launches, int* combines) {
  if (!attn_ms || !combine_ms || !launches || !combines) return MOLOT_EINVAL;
  std::lock_guard<std::mutex> lk(g_prof_mu);
  g_prof_on = false;
  double ta = 0.0, tc = 0.0;
  int n = 0, nc = 0, st = 0;
  for (ProfRec& r : g_prof) {
    if (!r.a0 || !r.a1 || (r.combine && (!r.c0 || !r.c1))) {
      st = (int)hipErrorInvalidValue;
      continue;
    }
    hipError_t e = hipEventSynchronize(r.combine ? r.c1 : r.a1);
    float ms = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, r.a0, r.a1);
    if (e != hipSuccess) {
      st = (int)e;
      continue;
    }
    ta += ms;
    ++n;
    if (r.combine) {
      e = hipEventElapsedTime(&ms, r.c0, r.c1);
      if (e != hipSuccess) {
        st = (int)e;
        continue;
      }
      tc += ms;
      ++nc;
    }
  }
  for (ProfRec& r : g_prof) prof_destroy(r);
  g_prof.clear();
  *attn_ms = (float)ta;
  *combine_ms = (float)tc;
  *launches = n;
  *combines = nc;
  return st;
}

void molot_hip_set_tuning(int wgs_per_cu) { g_wgs_per_cu = wgs_per_cu > 0 ? wgs_per_cu : 0; }

void molot_hip_set_merge(int in_launch) { g_merge = in_launch < 0 ? -1 : (in_launch ? 1 : 0); }

void molot_hip_set_prefill_presplit(int on) { g_presplit = on ? 1 : 0; }

int molot_hip_rope_apply(float* x, int nheads, int d, int pos, const float* inv_freq,
                         void* stream) {
  if (!x || !inv_freq || nheads < 0 || d <= 0 || (d & 1) || d > 2048) return MOLOT_EINVAL;
  if (nheads == 0) return 0;
  RopeArgs a{};
  a.q = x;
  a.inv_freq = inv_freq;
  a.nq = nheads;
  a.d = d;
  a.pos = pos;
  hipLaunchKernelGGL(rope_append_kernel, dim3(nheads, 1), dim3(((d / 2) + 63) / 64 * 64), 0,
                     (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

static int rope_append_impl(float* q, const float* k_new, const float* v_new, void* K, void* V,
                            int nq, int nkv, int d, int slot, int pos, const float* inv_freq,
                            int kv_dtype, const Norms& nm, void* stream) {
  if (nq < 0 || nkv <= 0 || d <= 0 || (d & 1) || d > 2048 || slot < 0) return MOLOT_EINVAL;
  if (!norms_ok(nm)) return MOLOT_EINVAL;
  if ((nq > 0 && !q) || !k_new || !v_new || !K || !V) return MOLOT_EINVAL;
  if (!valid_kv(kv_dtype)) return MOLOT_EINVAL;
  // rows only the attention kernels can read back (their Q8 head dims)
  if (kv_dtype == MOLOT_KV_Q8 && check_common(nkv, nkv, d, kv_dtype)) return MOLOT_ENOTSUP;
  RopeArgs a{};
  a.q = q;
  a.k_new = k_new;
  a.v_new = v_new;
  a.K = K;
  a.V = V;
  a.inv_freq = inv_freq;
  token_major(a, nkv, d, kv_dtype);
  a.nq = nq;
  a.nkv = nkv;
  a.d = d;
  a.slot = slot;
  a.pos = pos;
  a.kv_dtype = kv_dtype;
  a.append = 1;
  a.q_norm = nm.q;
  a.k_norm = nm.k;
  a.v_norm = nm.v;
  a.eps = nm.eps;
  hipLaunchKernelGGL(rope_append_kernel, dim3(nq + nkv, 1), dim3(((d / 2) + 63) / 64 * 64), 0,
                     (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

int molot_hip_rope_append(float* q, const float* k_new, const float* v_new, void* K, void* V,
                          int nq, int nkv, int d, int slot, int pos, const float* inv_freq,
                          int kv_dtype, void* stream) {
  return rope_append_impl(q, k_new, v_new, K, V, nq, nkv, d, slot, pos, inv_freq, kv_dtype,
                          Norms{}, stream);
}

int molot_hip_attn_decode_strided(const float* Q, const void* K, const void* V, float* O, int nq,
                                  int nkv, int n, int d, int64_t tok_stride, int64_t head_stride,
                                  float scale, int pos_cur, int window, int kv_dtype,
                                  void* stream) {
  int st = check_common(nq, nkv, d, kv_dtype);
  if (st) return st;
  if (!Q || !O || n < 0) return MOLOT_EINVAL;
  if (kv_dtype == MOLOT_KV_Q8 && (tok_stride != q8_row_bytes(nkv, d) || head_stride != d))
    return MOLOT_EINVAL;  // Q8: the token-major byte layout only
  int t0 = (window > 0 && pos_cur - window + 1 > 0) ? pos_cur - window + 1 : 0;
  if (t0 > n) t0 = n;
  const int n_att = n - t0;
  if (n_att <= 0) return zero_out(O, (int64_t)nq * d, (hipStream_t)stream);  // o = 0
  if (!K || !V) return MOLOT_EINVAL;
  const int esz = kv_esz(kv_dtype);
  // Rows the kernels can load: at the kernels' head dims (64, 128, 256,
  // 512) 16-byte vectors, so 16-byte aligned row starts; at a padded head
  // dim two-element pieces, so even strides.  A Q8 cache has the fixed
  // layout checked above, whose padded head dims load 4-code pieces.
  const bool padded = d != 64 && d != 128 && d != 256 && d != 512;
  const bool rows_ok = kv_dtype == MOLOT_KV_Q8 ||
                       (padded ? tok_stride % 2 == 0 && head_stride % 2 == 0
                               : (tok_stride * esz) % 16 == 0 && (head_stride * esz) % 16 == 0);
  if (!aligned16(K) || !aligned16(V) || !aligned16(Q) || !aligned16(O) || !rows_ok)
    return MOLOT_EINVAL;
  AttnArgs a{};
  a.q = Q;
  a.k = const_cast<void*>(K);
  a.v = const_cast<void*>(V);
  a.o = O;
  a.tok_stride = tok_stride;
  a.head_stride = head_stride;
  a.sc_off = (int64_t)nkv * d;  // Q8 scales after the row's codes
  a.sc_head = 4;
  a.nq = nq;
  a.nkv = nkv;
  a.n = n;
  a.t0 = t0;
  a.pos = pos_cur;
  a.window = window;
  a.scale = scale;
  return run_attn<false, false>(a, d, kv_dtype, n_att, 1, stream);
}

int molot_hip_attn_decode_gqa_cache(const float* Q, const void* K, const void* V, float* O,
                                    int nq, int nkv, int n, int qhd, float scale, int pos_cur,
                                    int window, int kv_dtype, void* stream) {
  const int64_t row = kv_dtype == MOLOT_KV_Q8 ? q8_row_bytes(nkv, qhd) : (int64_t)nkv * qhd;
  return molot_hip_attn_decode_strided(Q, K, V, O, nq, nkv, n, qhd, row, qhd, scale, pos_cur,
                                       window, kv_dtype, stream);
}

int molot_hip_attn_decode_gqa(const float* Q, const void* K, const void* V, float* O, int nq,
                              int nkv, int n, int d, float scale, int kv_dtype, void* stream) {
  return molot_hip_attn_decode_strided(Q, K, V, O, nq, nkv, n, d, d, (int64_t)n * d, scale, n, 0,
                                       kv_dtype, stream);
}

int molot_hip_attn_decode_gqa_win(const float* Q, const void* K, const void* V, float* O, int nq,
                                  int nkv, int n, int d, float scale, int pos_cur, int window,
                                  int kv_dtype, void* stream) {
  return molot_hip_attn_decode_strided(Q, K, V, O, nq, nkv, n, d, d, (int64_t)n * d, scale,
                                       pos_cur, window, kv_dtype, stream);
}

int molot_hip_attn_decode_head_win(const float* Q, const void* K, const void* V, float* out,
                                   int n, int d, float scale, int pos_cur, int window,
                                   int kv_dtype, void* stream) {
  return molot_hip_attn_decode_strided(Q, K, V, out, 1, 1, n, d, d, (int64_t)n * d, scale,
                                       pos_cur, window, kv_dtype, stream);
}

static int decode_step_impl(float* q, const float* k_new, const float* v_new, void* K, void* V,
                            float* O, int nq, int nkv, int d, int slot, int pos,
                            const float* inv_freq, float scale, int window, int kv_dtype,
                            const Norms& nm, void* stream, void* ext_ws = nullptr,
                            int64_t ext_ws_bytes = 0) {
  int st = check_common(nq, nkv, d, kv_dtype);
  if (st) return st;
  if (!norms_ok(nm)) return MOLOT_EINVAL;
  if (!q || !k_new || !v_new || !K || !V || !O || slot < 0) return MOLOT_EINVAL;
  if (!aligned16(K) || !aligned16(V) || !aligned16(q) || !aligned16(O)) return MOLOT_EINVAL;
  const int n = slot + 1;
  int t0 = (window > 0 && pos - window + 1 > 0) ? pos - window + 1 : 0;
  if (t0 > n) t0 = n;
  if (t0 > n - 1) {
    // the new token itself is outside the window: append, rotate q, o = 0
    st = rope_append_impl(q, k_new, v_new, K, V, nq, nkv, d, slot, pos, inv_freq, kv_dtype, nm,
                          stream);
    if (st) return st;
    return zero_out(O, (int64_t)nq * d, (hipStream_t)stream);
  }
  AttnArgs a{};
  a.q_norm = nm.q;
  a.k_norm = nm.k;
  a.v_norm = nm.v;
  a.eps = nm.eps;
  a.q = q;
  a.q_out = q;
  a.k_new = k_new;
  a.v_new = v_new;
  a.k = K;
  a.v = V;
  a.inv_freq = inv_freq;
  a.o = O;
  token_major(a, nkv, d, kv_dtype);
  a.nq = nq;
  a.nkv = nkv;
  a.n = n;
  a.t0 = t0;
  a.pos = pos;
  a.window = window;
  a.scale = scale;
  a.fold = 1;
  a.ext_ws = ext_ws;
  a.ext_ws_bytes = ext_ws_bytes;
  return run_attn<false, true>(a, d, kv_dtype, n - 1 - t0, 1, stream);  // cache rows
}

int molot_hip_decode_step(float* q, const float* k_new, const float* v_new, void* K, void* V,
                          float* O, int nq, int nkv, int d, int slot, int pos,
                          const float* inv_freq, float scale, int window, int kv_dtype,
                          void* stream) {
  return decode_step_impl(q, k_new, v_new, K, V, O, nq, nkv, d, slot, pos, inv_freq, scale,
                          window, kv_dtype, Norms{}, stream);
}

int molot_hip_decode_step_noalloc(float* q, const float* k_new, const float* v_new, void* K,
                                  void* V, float* O, int nq, int nkv, int d, int slot, int pos,
                                  const float* inv_freq, float scale, int window, int kv_dtype,
                                  void* stream) {
  void* ws = nullptr;
  const int st = noalloc_scratch(&ws);
  if (st) return st;
  return decode_step_impl(q, k_new, v_new, K, V, O, nq, nkv, d, slot, pos, inv_freq, scale,
                          window, kv_dtype, Norms{}, stream, ws, (int64_t)kScratchBytes);
}

int molot_hip_decode_step_norm(float* q, const float* k_new, const float* v_new, void* K,
                               void* V, float* O, int nq, int nkv, int d, int slot, int pos,
                               const float* q_norm, const float* k_norm, int v_norm, float eps,
                               const float* inv_freq, float scale, int window, int kv_dtype,
                               void* stream) {
  Norms nm;
  nm.q = q_norm;
  nm.k = k_norm;
  nm.v = v_norm ? 1 : 0;
  nm.eps = eps;
  return decode_step_impl(q, k_new, v_new, K, V, O, nq, nkv, d, slot, pos, inv_freq, scale,
                          window, kv_dtype, nm, stream);
}

static int paged_args(AttnArgs& a, const float* Q, void* K, void* V, float* O,
                      const int32_t* block_table, const int32_t* seq_lens, const int32_t* pos,
                      int B, int max_blocks, int max_seq_len, int nq, int nkv, int d, int page,
                      float scale, int window, int kv_dtype, int* span) {
  int st = check_common(nq, nkv, d, kv_dtype);
  if (st) return st;
  if (!Q || !K || !V || !O || !block_table || !seq_lens || B < 0 || max_blocks <= 0 ||
      max_seq_len < 0 || page <= 0 || (page & (page - 1)))
    return MOLOT_EINVAL;
  if ((int64_t)max_seq_len > (int64_t)max_blocks * page) return MOLOT_EINVAL;
  if (!aligned16(K) || !aligned16(V) || !aligned16(Q) || !aligned16(O)) return MOLOT_EINVAL;
  // head rows of the built dims are whole 16-byte vectors; other even dims
  // run padded, reading two-element pieces (4- or 8-byte aligned)
  if (!q8_pages_ok(nkv, page, kv_dtype)) return MOLOT_EINVAL;
  int shift = 0;
  while ((1 << shift) < page) ++shift;
  a.q = Q;
  a.k = K;
  a.v = V;
  a.o = O;
  a.block_table = block_table;
  a.seq_lens = seq_lens;
  a.pos_arr = pos;
  paged_layout(a, nkv, d, page, kv_dtype);
  a.nq = nq;
  a.nkv = nkv;
  a.max_blocks = max_blocks;
  a.page_shift = shift;
  a.window = window;
  a.scale = scale;
  // widest attended range of any sequence: with pos[] given, pos may lag the
  // cache end, so only max_seq_len bounds it
  *span = (!pos && window > 0 && window < max_seq_len) ? window : max_seq_len;
  return 0;
}

int molot_hip_attn_decode_paged(const float* Q, const void* K, const void* V, float* O,
                                const int32_t* block_table, const int32_t* seq_lens,
                                const int32_t* pos, int B, int max_blocks, int max_seq_len,
                                int nq, int nkv, int d, int page, float scale, int window,
                                int kv_dtype, void* stream) {
  AttnArgs a{};
  int span = 0;
  int st = paged_args(a, Q, const_cast<void*>(K), const_cast<void*>(V), O, block_table, seq_lens,
                      pos, B, max_blocks, max_seq_len, nq, nkv, d, page, scale, window, kv_dtype,
                      &span);
  if (st) return st;
  if (B == 0) return 0;
  return run_attn<true, false>(a, d, kv_dtype, span, B, stream);
}

static int rope_append_paged_impl(float* q, const float* k_new, const float* v_new, void* K,
                                  void* V, const int32_t* block_table, const int32_t* seq_lens,
                                  const int32_t* pos, int B, int max_blocks, int nq, int nkv,
                                  int d, int page, const float* inv_freq, int kv_dtype,
                                  const Norms& nm, void* stream);

static int decode_step_paged_impl(float* q, const float* k_new, const float* v_new, void* K,
                                  void* V, float* O, const int32_t* block_table,
                                  const int32_t* seq_lens, const int32_t* pos, int B,
                                  int max_blocks, int max_seq_len, int nq, int nkv, int d,
                                  int page, const float* inv_freq, float scale, int window,
                                  int kv_dtype, const Norms& nm, void* stream) {
  if (!norms_ok(nm)) return MOLOT_EINVAL;
  AttnArgs a{};
  int span = 0;
  int st = paged_args(a, q, K, V, O, block_table, seq_lens, pos, B, max_blocks, max_seq_len, nq,
                      nkv, d, page, scale, window, kv_dtype, &span);
  if (st) return st;
  if (!k_new || !v_new) return MOLOT_EINVAL;
  if (B == 0) return 0;
  if (pos) {
    // a position behind the cache end can leave the new slot outside the
    // window; the split path only folds in rows it attends, so take the
    // unfused kernels there (append, then attention over the cache)
    st = rope_append_paged_impl(q, k_new, v_new, K, V, block_table, seq_lens, pos, B,
                                max_blocks, nq, nkv, d, page, inv_freq, kv_dtype, nm, stream);
    if (st) return st;
    return run_attn<true, false>(a, d, kv_dtype, span, B, stream);
  }
  a.q_norm = nm.q;
  a.k_norm = nm.k;
  a.v_norm = nm.v;
  a.eps = nm.eps;
  a.q_out = q;
  a.k_new = k_new;
  a.v_new = v_new;
  a.inv_freq = inv_freq;
  a.fold = 1;
  return run_attn<true, true>(a, d, kv_dtype, span, B, stream);  // span >= cache rows
}

int molot_hip_decode_step_paged(float* q, const float* k_new, const float* v_new, void* K,
                                void* V, float* O, const int32_t* block_table,
                                const int32_t* seq_lens, const int32_t* pos, int B,
                                int max_blocks, int max_seq_len, int nq, int nkv, int d, int page,
                                const float* inv_freq, float scale, int window, int kv_dtype,
                                void* stream) {
  return decode_step_paged_impl(q, k_new, v_new, K, V, O, block_table, seq_lens, pos, B,
                                max_blocks, max_seq_len, nq, nkv, d, page, inv_freq, scale,
                                window, kv_dtype, Norms{}, stream);
}

int molot_hip_decode_step_paged_norm(float* q, const float* k_new, const float* v_new, void* K,
                                     void* V, float* O, const int32_t* block_table,
                                     const int32_t* seq_lens, const int32_t* pos, int B,
                                     int max_blocks, int max_seq_len, int nq, int nkv, int d,
                                     int page, const float* q_norm, const float* k_norm,
                                     int v_norm, float eps, const float* inv_freq, float scale,
                                     int window, int kv_dtype, void* stream) {
  Norms nm;
  nm.q = q_norm;
  nm.k = k_norm;
  nm.v = v_norm ? 1 : 0;
  nm.eps = eps;
  return decode_step_paged_impl(q, k_new, v_new, K, V, O, block_table, seq_lens, pos, B,
                                max_blocks, max_seq_len, nq, nkv, d, page, inv_freq, scale,
                                window, kv_dtype, nm, stream);
}

int molot_hip_rope_append_paged(float* q, const float* k_new, const float* v_new, void* K,
                                void* V, const int32_t* block_table, const int32_t* seq_lens,
                                const int32_t* pos, int B, int max_blocks, int nq, int nkv, int d,
                                int page, const float* inv_freq, int kv_dtype, void* stream) {
  return rope_append_paged_impl(q, k_new, v_new, K, V, block_table, seq_lens, pos, B, max_blocks,
                                nq, nkv, d, page, inv_freq, kv_dtype, Norms{}, stream);
}

static int rope_append_paged_impl(float* q, const float* k_new, const float* v_new, void* K,
                                  void* V, const int32_t* block_table, const int32_t* seq_lens,
                                  const int32_t* pos, int B, int max_blocks, int nq, int nkv,
                                  int d, int page, const float* inv_freq, int kv_dtype,
                                  const Norms& nm, void* stream) {
  if (!norms_ok(nm)) return MOLOT_EINVAL;
  if (nq < 0 || nkv <= 0 || d <= 0 || (d & 1) || d > 2048 || B < 0 || max_blocks <= 0 ||
      page <= 0)
    return MOLOT_EINVAL;
  if ((nq > 0 && !q) || !k_new || !v_new || !K || !V || !block_table || !seq_lens)
    return MOLOT_EINVAL;
  if (!valid_kv(kv_dtype)) return MOLOT_EINVAL;
  // the page layout every paged attention entry accepts
  if ((page & (page - 1)) || !q8_pages_ok(nkv, page, kv_dtype)) return MOLOT_EINVAL;
  if (kv_dtype == MOLOT_KV_Q8 && check_common(nkv, nkv, d, kv_dtype)) return MOLOT_ENOTSUP;
  if (B == 0) return 0;
  RopeArgs a{};
  a.q = q;
  a.k_new = k_new;
  a.v_new = v_new;
  a.K = K;
  a.V = V;
  a.inv_freq = inv_freq;
  a.block_table = block_table;
  a.seq_lens = seq_lens;
  a.pos_arr = pos;
  paged_layout(a, nkv, d, page, kv_dtype);
  a.nq = nq;
  a.nkv = nkv;
  a.d = d;
  a.max_blocks = max_blocks;
  a.page = page;
  a.kv_dtype = kv_dtype;
  a.append = 1;
  a.q_norm = nm.q;
  a.k_norm = nm.k;
  a.v_norm = nm.v;
  a.eps = nm.eps;
  hipLaunchKernelGGL(rope_append_kernel, dim3(nq + nkv, B), dim3(((d / 2) + 63) / 64 * 64), 0,
                     (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

// The attended keys of a prefill: [T0, N) with T0 the window start of its
// first query (pos0), split into 16-bit pieces once per launch for fp32 and
// Q8 caches when the pieces fit (kMaxPiecesBytes) and the workspace need not
// grow under capture.  Returns the pieces buffer (NULL: the attention kernel
// splits each staged tile itself) and sets T0 and R.
// only: the launch has no per-tile kernel (a Q8 cache at d = 256): the
// pieces are made whatever the presplit switch says (within the same cap;
// past it, or under a capture that would grow them, such a prefill runs as
// prefill rows).
static int prefill_pieces(int nkv, int N, int d, int pos0, int window, int kv_dtype, void* stream,
                          void** ws, int* T0, int64_t* R, bool only = false) {
  *ws = nullptr;
  *T0 = window > 0 && pos0 - window + 1 > 0 ? std::min(pos0 - window + 1, N) : 0;
  *R = (int64_t)N - *T0;
  if (!only && (kv_dtype == MOLOT_KV_BF16 || !g_presplit.load(std::memory_order_relaxed))) return 0;
  const size_t need = (size_t)2 * nkv * 3 * *R * d * sizeof(uint16_t);
  void* p = nullptr;
  const int st =
      *R > 0 && need <= kMaxPiecesBytes ? pieces_workspace(stream, need, &p) : MOLOT_ENOWS;
  if (st && st != MOLOT_ENOWS) return st;
  if (!st) *ws = p;
  return 0;
}

// The prefill at a head dim the matrix-core prefill cannot tile (d = 512:
// its three q pieces alone would take 192 registers a lane and a 32-key tile
// of K and V pieces 192 KB of LDS; an even d that is not a multiple of 8):
// the vector-ALU decode kernel with each query row as a sequence of its own
// (AttnArgs::pf) over the one cache, contiguous or through the prompt's
// block-table row.  Each query row streams its attended rows; neighbouring
// rows of a prompt read the same keys, which the L2 and the Infinity Cache
// serve after the first.
static int prefill_rows(const float* Qm, const void* K, const void* V, float* Om, int nq,
                        int nkv, int M, int N, int d, float scale, int pos0, int window,
                        int kv_dtype, const int32_t* block_row, int page, void* stream) {
  if ((int64_t)M > 65535) return MOLOT_ENOTSUP;  // grid rows: one per query
  AttnArgs a{};
  a.q = Qm;
  a.k = const_cast<void*>(K);
  a.v = const_cast<void*>(V);
  a.o = Om;
  if (block_row) {
    if (page <= 0 || (page & (page - 1)) || !q8_pages_ok(nkv, page, kv_dtype)) return MOLOT_EINVAL;
    paged_layout(a, nkv, d, page, kv_dtype);
    a.block_table = block_row;
    a.max_blocks = 0;  // every row reads the one block-table row
    while ((1 << a.page_shift) < page) ++a.page_shift;
  } else {
    token_major(a, nkv, d, kv_dtype);
  }
  a.nq = nq;
  a.nkv = nkv;
  a.n = N;
  a.pos = pos0;
  a.window = window;
  a.scale = scale;
  a.pf = 1;
  // the widest attended range of any query row
  const int span = window > 0 && window < N ? window : N;
  return block_row ? run_attn<true, false>(a, d, kv_dtype, span, M, stream)
                   : run_attn<false, false>(a, d, kv_dtype, span, M, stream);
}

// split_rows: rows of [T0, N) pf_split_kernel still has to split (the
// appending step wrote the pieces of the others; -1: all of them)
static int attn_prefill_impl(const float* Qm, const void* K, const void* V, float* Om, int nq,
                             int nkv, int M, int N, int d, float scale, int pos0, int window,
                             int kv_dtype, const int32_t* block_row, int page, void* stream,
                             int split_rows = -1) {
  int st = check_common(nq, nkv, d, kv_dtype);
  if (st) return st;
  // The prefill kernels are built for D = 64, 128, 256.  Any other head dim
  // that is a multiple of 8 below 256 (fp32 or bf16) runs padded to the next
  // D: the split kernel and the per-tile loads read each row at its stored
  // length d and fill the columns past it with 0, q is read and O written
  // at d.  A Q8 cache at d = 256 runs only through the pieces (the kernel
  // that splits staged Q8 tiles itself is built for 64 and 128).  Head dims
  // above 256 and even ones that are not multiples of 8 run as prefill rows
  // (prefill_rows).
  const bool padded = !supported_d(d);
  // Q8 caches at padded dims too (the matrix-core prefill reads whole
  // 16-code chunks of the built dims only)
  const bool rows_path = d > 256 || d % 8 != 0 || (padded && kv_dtype == MOLOT_KV_Q8);
  const bool pieces_only = kv_dtype == MOLOT_KV_Q8 && d == 256;
  const int D = padded ? (d <= 64 ? 64 : d <= 128 ? 128 : 256) : d;
  if (M < 0 || N < 0 || pos0 < 0 || (M > 0 && (!Qm || !Om))) return MOLOT_EINVAL;
  if (M == 0) return 0;
  if (N == 0) return zero_out(Om, (int64_t)M * nq * d, (hipStream_t)stream);
  if (!K || !V || !aligned16(K) || !aligned16(V) || !aligned16(Qm) || !aligned16(Om))
    return MOLOT_EINVAL;
  if (rows_path)
    return prefill_rows(Qm, K, V, Om, nq, nkv, M, N, d, scale, pos0, window, kv_dtype, block_row,
                        page, stream);
  const int64_t rows = (int64_t)M * (nq / nkv);
  auto nqb_of = [&](int w) { return (rows + 16 * w - 1) / (16 * w); };
  int pw = kPfWaves;
  int64_t nqb = nqb_of(pw);
  // A grid of fewer workgroups than CUs (few query rows over a long cache,
  // e.g. a prompt chunk after a long context) splits each query block's key
  // tiles over nsplit workgroups, at least 4 tiles each, and combine_kernel
  // merges their partials (slots: one query row of one head).
  int nsplit = 1;
  float* part = nullptr;
  if (nqb * nkv < num_cus() && (int64_t)M * nq <= 65535) {
    const int last = pos0 + M - 1;  // the query attending the most keys
    const int t0l = window > 0 && last - window + 1 > 0 ? std::min(last - window + 1, N) : 0;
    const int64_t tiles = (std::min(last + 1, N) - t0l + 31) / 32;
    const int64_t want = (num_cus() + nqb * nkv - 1) / (nqb * nkv);
    nsplit = (int)std::max<int64_t>(1, std::min<int64_t>({16, want, tiles / 4}));
    if (nsplit > 1) {
      unsigned long long* ctr = nullptr;
      void* ws = nullptr;
      st = workspace(stream, sizeof(float) * (size_t)M * nq * nsplit * (D + 2), &ctr, &ws);
      if (st && st != MOLOT_ENOWS) return st;
      if (st) nsplit = 1;  // under capture the workspace cannot grow
      else part = reinterpret_cast<float*>(ws);
      st = 0;
    }
  }
  if (nsplit == 1 && pw == 8 && nqb * nkv < num_cus()) {
    pw = 4;  // no split: twice the workgroups on 4 waves
    nqb = nqb_of(4);
  }
  const int pf_threads = 64 * pw;
  if (nqb * nkv * nsplit > (int64_t)0x7FFFFFFF) return MOLOT_ENOTSUP;
  PfArgs a{};
  a.q = Qm;
  a.k = K;
  a.v = V;
  a.o = Om;
  a.nq = nq;
  a.nkv = nkv;
  a.M = M;
  a.N = N;
  a.pos0 = pos0;
  a.window = window;
  a.nqb = (int)nqb;
  a.scale = scale;
  a.block_table = block_row;
  a.nsplit = nsplit;
  a.part_o = part;
  a.part_ml = part ? part + (size_t)M * nq * nsplit * D : nullptr;
  a.dh = d;
  if (block_row) {
    if (page <= 0 || (page & (page - 1)) || !q8_pages_ok(nkv, page, kv_dtype))
      return MOLOT_EINVAL;
    while ((1 << a.page_shift) < page) ++a.page_shift;
  }
  PfFn pk = pieces_only ? nullptr : pf_kernel(D, kv_dtype, block_row != nullptr, pw);
  if (!pk && !pieces_only) return MOLOT_ENOTSUP;
  // fp32 and Q8 caches: split the attended keys into 16-bit pieces once
  // (pf_split_kernel), and let the attention kernel copy them into LDS.
  // Every query attends keys in [t0(query 0), N).  Not under stream capture
  // when the workspace would have to grow, nor past kMaxPiecesBytes: the
  // kernel then splits each staged tile itself.
  {
    void* ws = nullptr;
    int T0 = 0;
    int64_t R = 0;
    st = prefill_pieces(nkv, N, D, pos0, window, kv_dtype, stream, &ws, &T0, &R, pieces_only);
    if (st) return st;
    if (!ws && pieces_only) {
      if (R == 0) return zero_out(Om, (int64_t)M * nq * d, (hipStream_t)stream);  // no key attended
      // a capture that would have to grow them, or past the cap: the vector-
      // ALU kernel reads the Q8 rows itself
      return prefill_rows(Qm, K, V, Om, nq, nkv, M, N, d, scale, pos0, window, kv_dtype,
                          block_row, page, stream);
    }
    if (ws) {
      a.pieces = reinterpret_cast<const uint16_t*>(ws);
      a.T0 = T0;
      a.R = (int)R;
      a.Rsplit = split_rows < 0 ? (int)R : (int)std::min<int64_t>(split_rows, R);
      if (a.Rsplit > 0) {
        const int64_t units = (int64_t)a.Rsplit * (D / 8);
        hipLaunchKernelGGL(pf_split(D, kv_dtype, block_row != nullptr),
                           dim3((unsigned)((units + 255) / 256), nkv, 2), dim3(256), 0,
                           (hipStream_t)stream, a, reinterpret_cast<uint16_t*>(ws));
        st = (int)hipGetLastError();
        if (st) return st;
      }
      pk = pf_kernel_pre(D, pw);
    }
  }
  const dim3 grid((unsigned)(nqb * nkv * nsplit));
  CombArgs cb{};  // split-K: (token, q head) rows as slots of one head each
  cb.part_o = a.part_o;
  cb.part_ml = a.part_ml;
  cb.o = Om;
  cb.nq = nq;
  cb.nkv = nq;
  cb.gh = 1;
  cb.nsub = 1;
  cb.d = D;
  cb.dh = d;
  cb.nchunks = nsplit;
  cb.chunk = 1;
  cb.pairs = comb_pairs(nsplit);
  // at most 8 splits: the row merge, one wave per 64V outputs of a slot
  // (2048 tokens x 8 q heads at d = 256 over 2 splits: 9.2 us, against 22.2
  // with a wave per 64 outputs and 82 us on combine_kernel's 4 workgroups a
  // slot); more splits: combine_kernel
  const bool cwave = nsplit <= 8;
  const int cv = D % 256 == 0 ? 4 : (D % 128 == 0 ? 2 : 1);
  const int64_t cunits = (int64_t)M * nq * (D / (64 * cv));
  using RowsFn = void (*)(CombArgs, int64_t);
  const RowsFn rk = nsplit <= 4 ? (cv == 4 ? combine_rows_kernel<4, 4>
                                  : cv == 2 ? combine_rows_kernel<4, 2> : combine_rows_kernel<4, 1>)
                                : (cv == 4 ? combine_rows_kernel<8, 4>
                                  : cv == 2 ? combine_rows_kernel<8, 2> : combine_rows_kernel<8, 1>);
  const dim3 cgrid = cwave ? dim3((unsigned)((cunits + 3) / 4))
                           : dim3((unsigned)((int64_t)M * nq), (unsigned)(D / cb.pairs));
  const dim3 cblock = cwave ? dim3((unsigned)kCombWaveThreads) : dim3(kCombThreads);
  const size_t clds = cwave ? 0 : sizeof(float) * (size_t)comb_lds_floats(nsplit);
  std::lock_guard<std::mutex> plk(g_prof_mu);
  if (prof_active(stream)) {
    ProfRec pr{prof_event(), prof_event(), nullptr, nullptr, nsplit > 1};
    hipExtLaunchKernelGGL(pk, grid, dim3(pf_threads), 0, (hipStream_t)stream, pr.a0, pr.a1, 0, a);
    st = (int)hipGetLastError();
    if (!st && nsplit > 1) {
      pr.c0 = prof_event();
      pr.c1 = prof_event();
      if (cwave)
        hipExtLaunchKernelGGL(rk, cgrid, cblock, 0, (hipStream_t)stream, pr.c0, pr.c1, 0, cb,
                              cunits);
      else
        hipExtLaunchKernelGGL(combine_kernel, cgrid, cblock, clds, (hipStream_t)stream, pr.c0,
                              pr.c1, 0, cb);
      st = (int)hipGetLastError();
    }
    g_prof.push_back(pr);
    return st;
  }
  hipLaunchKernelGGL(pk, grid, dim3(pf_threads), 0, (hipStream_t)stream, a);
  st = (int)hipGetLastError();
  if (st || nsplit == 1) return st;
  if (cwave)
    hipLaunchKernelGGL(rk, cgrid, cblock, 0, (hipStream_t)stream, cb, cunits);
  else
    hipLaunchKernelGGL(combine_kernel, cgrid, cblock, clds, (hipStream_t)stream, cb);
  return (int)hipGetLastError();
}

int molot_hip_attn_prefill_gqa(const float* Qm, const void* K, const void* V, float* Om, int nq,
                               int nkv, int M, int N, int d, float scale, int pos0, int window,
                               int kv_dtype, void* stream) {
  return attn_prefill_impl(Qm, K, V, Om, nq, nkv, M, N, d, scale, pos0, window, kv_dtype,
                           nullptr, 0, stream);
}

static int prefill_step_impl(float* q, const float* k_new, const float* v_new, void* K, void* V,
                             float* O, int nq, int nkv, int d, int M, int slot0, int pos0,
                             const float* q_norm, const float* k_norm, int v_norm, float eps,
                             const float* inv_freq, float scale, int window, int kv_dtype,
                             const int32_t* block_row, int page, int max_blocks, void* stream) {
  int st = check_common(nq, nkv, d, kv_dtype);
  if (st) return st;
  // the prefill kernels' head dims, a multiple of 8 below 256 run padded, or
  // prefill rows (d > 256, not a multiple of 8, or a padded Q8 cache; see
  // attn_prefill_impl)
  const bool pieces_only = kv_dtype == MOLOT_KV_Q8 && d == 256;  // no per-tile kernel
  Norms nm;
  nm.q = q_norm;
  nm.k = k_norm;
  nm.v = v_norm ? 1 : 0;
  nm.eps = eps;
  if (!norms_ok(nm) || M < 0 || slot0 < 0 || pos0 < 0) return MOLOT_EINVAL;
  if (M == 0) return 0;
  if (!q || !k_new || !v_new || !K || !V || !O) return MOLOT_EINVAL;
  if ((int64_t)M > 65535) return MOLOT_ENOTSUP;  // one grid row per token
  if (block_row && ((int64_t)slot0 + M > (int64_t)max_blocks * page || page <= 0 ||
                    (page & (page - 1)) || !q8_pages_ok(nkv, page, kv_dtype)))
    return MOLOT_EINVAL;
  RopeArgs r{};
  r.q = q;
  r.k_new = k_new;
  r.v_new = v_new;
  r.K = K;
  r.V = V;
  r.inv_freq = inv_freq;
  if (block_row) {  // every token of the one sequence through its block-table row
    r.block_table = block_row;
    r.max_blocks = 0;
    r.page = page;
    paged_layout(r, nkv, d, page, kv_dtype);
  } else {
    token_major(r, nkv, d, kv_dtype);
  }
  r.nq = nq;
  r.nkv = nkv;
  r.d = d;
  r.slot = slot0;
  r.pos = pos0;
  r.kv_dtype = kv_dtype;
  r.append = 1;
  r.tokens = 1;
  r.q_norm = nm.q;
  r.k_norm = nm.k;
  r.v_norm = nm.v;
  r.eps = nm.eps;
  // the appended rows leave their pieces as they are stored; the split
  // kernel then covers only the cached rows before them, and a fresh prompt
  // needs no split launch (eager steps of 2048-token prompts: 32q/8kv/d128
  // fp32 252 -> 249 us, 8q/4kv/d256 window 1024 164.7 -> 161.6 us)
  void* pws = nullptr;
  int T0 = 0;
  int64_t R = 0;
  int split_rows = -1;
  if (supported_d(d)) {
    st = prefill_pieces(nkv, slot0 + M, d, pos0, window, kv_dtype, stream, &pws, &T0, &R,
                        pieces_only);
    if (st) return st;
    if (pws) {
      r.pieces = reinterpret_cast<uint16_t*>(pws);
      r.pc_T0 = T0;
      r.pc_R = (int)R;
      split_rows = std::max(0, slot0 - T0);
    }
  }
  st = launch_rope_tok(r, M, stream);
  if (st) return st;
  return attn_prefill_impl(q, K, V, O, nq, nkv, M, slot0 + M, d, scale, pos0, window, kv_dtype,
                           block_row, page, stream, split_rows);
}

int molot_hip_prefill_step(float* q, const float* k_new, const float* v_new, void* K, void* V,
                           float* O, int nq, int nkv, int d, int M, int slot0, int pos0,
                           const float* q_norm, const float* k_norm, int v_norm, float eps,
                           const float* inv_freq, float scale, int window, int kv_dtype,
                           void* stream) {
  return prefill_step_impl(q, k_new, v_new, K, V, O, nq, nkv, d, M, slot0, pos0, q_norm, k_norm,
                           v_norm, eps, inv_freq, scale, window, kv_dtype, nullptr, 0, 0, stream);
}

int molot_hip_prefill_step_paged(float* q, const float* k_new, const float* v_new, void* K,
                                 void* V, float* O, const int32_t* block_row, int max_blocks,
                                 int page, int nq, int nkv, int d, int M, int slot0, int pos0,
                                 const float* q_norm, const float* k_norm, int v_norm, float eps,
                                 const float* inv_freq, float scale, int window, int kv_dtype,
                                 void* stream) {
  if (!block_row || max_blocks <= 0) return MOLOT_EINVAL;
  return prefill_step_impl(q, k_new, v_new, K, V, O, nq, nkv, d, M, slot0, pos0, q_norm, k_norm,
                           v_norm, eps, inv_freq, scale, window, kv_dtype, block_row, page,
                           max_blocks, stream);
}

// Norm and RoPE of M rows of queries [M][nq][d] at positions pos0 + m, in
// place, no append (the RoPE/append kernel with its KV part off).
static int q_prologue(float* q, int nq, int d, int M, int pos0, const float* q_norm, float eps,
                      const float* inv_freq, void* stream) {
  if (nq < 0 || M < 0 || d <= 0 || (d & 1) || d > 2048 || pos0 < 0) return MOLOT_EINVAL;
  if (!(eps >= 0.f && eps < INFINITY)) return MOLOT_EINVAL;
  if (nq == 0 || M == 0) return 0;
  if (!q) return MOLOT_EINVAL;
  if ((int64_t)M > 65535) return MOLOT_ENOTSUP;  // one grid row per token
  if (!q_norm && !inv_freq) return 0;            // nothing to apply
  RopeArgs r{};
  r.q = q;
  r.inv_freq = inv_freq;
  r.nq = nq;
  r.nkv = 1;
  r.d = d;
  r.pos = pos0;
  r.tokens = 1;
  r.q_norm = q_norm;
  r.eps = eps;
  return launch_rope_tok(r, M, stream);
}

int molot_hip_prefill_q(float* q, int nq, int d, int M, int pos0, const float* q_norm, float eps,
                        const float* inv_freq, void* stream) {
  return q_prologue(q, nq, d, M, pos0, q_norm, eps, inv_freq, stream);
}

int molot_hip_decode_step_shared(float* q, const void* K, const void* V, float* O, int nq,
                                 int nkv, int d, int n, int pos, const float* q_norm, float eps,
                                 const float* inv_freq, float scale, int window, int kv_dtype,
                                 void* stream) {
  int st = check_common(nq, nkv, d, kv_dtype);
  if (st) return st;
  if (!q || !K || !V || !O || n <= 0 || pos < 0) return MOLOT_EINVAL;  // n = 0: forward.h:580
  if (!(eps >= 0.f && eps < INFINITY)) return MOLOT_EINVAL;
  if (!aligned16(K) || !aligned16(V) || !aligned16(q) || !aligned16(O)) return MOLOT_EINVAL;
  int t0 = (window > 0 && pos - window + 1 > 0) ? pos - window + 1 : 0;
  if (t0 >= n) {  // nothing attended: q still gets its norm and RoPE, o = 0
    st = q_prologue(q, nq, d, 1, pos, q_norm, eps, inv_freq, stream);
    if (st) return st;
    return zero_out(O, (int64_t)nq * d, (hipStream_t)stream);
  }
  AttnArgs a{};
  a.q = q;
  a.q_out = q;
  a.k = const_cast<void*>(K);
  a.v = const_cast<void*>(V);
  a.inv_freq = inv_freq;
  a.o = O;
  token_major(a, nkv, d, kv_dtype);
  a.nq = nq;
  a.nkv = nkv;
  a.n = n;
  a.t0 = t0;
  a.pos = pos;
  a.window = window;
  a.scale = scale;
  a.q_norm = q_norm;
  a.eps = eps;
  a.fold = 0;  // all n slots are the source layer's; nothing appended
  return run_attn<false, true>(a, d, kv_dtype, n - t0, 1, stream);
}

int molot_hip_decode_step_paged_shared(float* q, const void* K, const void* V, float* O,
                                       const int32_t* block_table, const int32_t* seq_lens,
                                       const int32_t* pos, int B, int max_blocks, int max_seq_len,
                                       int nq, int nkv, int d, int page, const float* q_norm,
                                       float eps, const float* inv_freq, float scale, int window,
                                       int kv_dtype, void* stream) {
  if (!(eps >= 0.f && eps < INFINITY)) return MOLOT_EINVAL;
  AttnArgs a{};
  int span = 0;
  int st = paged_args(a, q, const_cast<void*>(K), const_cast<void*>(V), O, block_table, seq_lens,
                      pos, B, max_blocks, max_seq_len, nq, nkv, d, page, scale, window, kv_dtype,
                      &span);
  if (st) return st;
  if (B == 0) return 0;
  a.q_out = q;
  a.inv_freq = inv_freq;
  a.q_norm = q_norm;
  a.eps = eps;
  a.fold = 0;
  return run_attn<true, true>(a, d, kv_dtype, span, B, stream);
}

int molot_hip_attn_prefill_paged(const float* Qm, const void* K, const void* V, float* Om,
                                 const int32_t* block_row, int max_blocks, int page, int nq,
                                 int nkv, int M, int N, int d, float scale, int pos0, int window,
                                 int kv_dtype, void* stream) {
  if (!block_row || max_blocks <= 0 || N < 0 || (int64_t)N > (int64_t)max_blocks * page)
    return MOLOT_EINVAL;
  return attn_prefill_impl(Qm, K, V, Om, nq, nkv, M, N, d, scale, pos0, window, kv_dtype,
                           block_row, page, stream);
}

int molot_hip_vexp(const float* x, float* y, int64_t n, void* stream) {
  if (n < 0 || (n > 0 && (!x || !y))) return MOLOT_EINVAL;
  if (n == 0) return 0;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(vexp_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, x,
                     y, n);
  return (int)hipGetLastError();
}

int molot_hip_prob_exp(const float* x, float* y, int64_t n, void* stream) {
  if (n < 0 || (n > 0 && (!x || !y))) return MOLOT_EINVAL;
  if (n == 0) return 0;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(prob_exp_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     x, y, n);
  return (int)hipGetLastError();
}

}  // extern "C"
