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
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <mutex>
#include <utility>

#include "molot_amd/attn_hip.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

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

template <typename T>
__device__ __forceinline__ typename KVT<T>::vec load16(const T* p) {
  return *reinterpret_cast<const typename KVT<T>::vec*>(p);
}

// Round-to-nearest-even fp32 -> bf16 (include/molot/quant.h:192-198).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
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

template <int N>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (N >= 2) v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  if constexpr (N >= 4) v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  if constexpr (N >= 8) v += dpp_f<0x141>(v);  // row_half_mirror
  if constexpr (N >= 16) v += dpp_f<0x140>(v); // row_mirror
  if constexpr (N >= 32) v += __shfl_xor(v, 16);
  if constexpr (N >= 64) v += __shfl_xor(v, 32);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

// exp used by the softmax (full-accuracy device expf).
__device__ __forceinline__ float softmax_exp(float x) { return expf(x); }

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
  int64_t tok_stride, head_stride, block_stride;
  int nq, nkv, d, slot, pos, max_blocks, page, kv_dtype, append;
};

// One workgroup per (head of q or k, sequence); one thread per rotation pair.
// Angle is the fp32 product pos*inv_freq[i] (include/molot/attn.h:22); its
// sine and cosine are evaluated in double and rounded, i.e. a full-range,
// correctly rounded (barring double rounding) fp32 sin/cos.
__global__ void rope_append_kernel(RopeArgs a) {
  const int hh = blockIdx.x;
  const int b = blockIdx.y;
  const int half = a.d >> 1;
  const int i = threadIdx.x;
  if (i >= half) return;
  int pos = a.pos;
  int slot = a.slot;
  if (a.seq_lens) {
    slot = a.seq_lens[b] - 1;
    pos = a.pos_arr ? a.pos_arr[b] : slot;
  }
  const float ang = (float)pos * a.inv_freq[i];
  double sd, cd;
  sincos((double)ang, &sd, &cd);
  const float c = (float)cd, s = (float)sd;
  if (hh < a.nq) {
    if (!a.q) return;
    float* x = a.q + ((int64_t)b * a.nq + hh) * a.d;
    const float x0 = x[i], x1 = x[i + half];
    x[i] = x0 * c - x1 * s;
    x[i + half] = x0 * s + x1 * c;
    return;
  }
  if (!a.append) return;
  const int kh = hh - a.nq;
  const float* kx = a.k_new + ((int64_t)b * a.nkv + kh) * a.d;
  const float* vx = a.v_new + ((int64_t)b * a.nkv + kh) * a.d;
  const float k0 = kx[i], k1 = kx[i + half];
  const float r0 = k0 * c - k1 * s;
  const float r1 = k0 * s + k1 * c;
  int64_t off;
  if (a.block_table) {
    const int64_t blk = a.block_table[(int64_t)b * a.max_blocks + slot / a.page];
    off = blk * a.block_stride + (int64_t)kh * a.head_stride + (int64_t)(slot % a.page) * a.tok_stride;
  } else {
    off = (int64_t)slot * a.tok_stride + (int64_t)kh * a.head_stride;
  }
  if (a.kv_dtype == MOLOT_KV_F32) {
    float* kd = (float*)a.K + off;
    float* vd = (float*)a.V + off;
    kd[i] = r0;
    kd[i + half] = r1;
    vd[i] = vx[i];
    vd[i + half] = vx[i + half];
  } else {
    uint16_t* kd = (uint16_t*)a.K + off;
    uint16_t* vd = (uint16_t*)a.V + off;
    kd[i] = f32_to_bf16(r0);
    kd[i + half] = f32_to_bf16(r1);
    vd[i] = f32_to_bf16(vx[i]);
    vd[i + half] = f32_to_bf16(vx[i + half]);
  }
}

// ---------------------------------------------------------------------------
// Split-K attention.
struct SplitArgs {
  const float* q;  // [B][nq][D]
  const void* k;
  const void* v;
  float* o;        // [B][nq][D]  (written directly when `direct`)
  float* part_o;   // [B][nq][nchunks][D]
  float* part_ml;  // [B][nq][nchunks][2] = (chunk max, chunk sum)
  const int32_t* block_table;
  const int32_t* seq_lens;
  const int32_t* pos_arr;
  int64_t tok_stride, head_stride, block_stride;
  int nq, nkv, n, t0, chunk, nchunks, max_blocks, page_shift, window, direct;
  float scale;
};

// Lanes cooperating on one K row in the score loop: enough that the query
// registers (GH heads x D/LPR elements) stay at <= 64, and at least 8 so a
// lane group reads >= 128 contiguous bytes per load.
template <int D, int GH, typename T>
constexpr int qk_lpr() {
  constexpr int VW = KVT<T>::VW;
  int l = 8;
  while (l * 64 < D * GH) l *= 2;
  if (l > D / VW) l = D / VW;
  return l;
}

template <int D, int GH, typename T, int NW>
struct SplitCfg {
  static constexpr int VW = KVT<T>::VW;
  static constexpr int LPR = qk_lpr<D, GH, T>();  // lanes per K row (scores)
  static constexpr int NV = D / (LPR * VW);       // 16-byte vectors per lane per row
  static constexpr int EPL = NV * VW;             // elements per lane per row
  static constexpr int RPS = 64 / LPR;            // rows per wave per step (scores)
  static constexpr int LPR2 = D / VW;             // lanes per V row (PV)
  static constexpr int RPI = 64 / LPR2;           // rows per wave per step (PV)
  static constexpr int UQK = NV >= 4 ? 2 : (NV == 2 ? 4 : 8);  // score steps in flight
  static constexpr int UPV = 8;                                // PV steps in flight
  static_assert(NV >= 1 && D % (LPR * VW) == 0, "bad score mapping");
  static_assert(LPR2 <= 64 && 64 % LPR2 == 0, "bad PV mapping");
};

template <int D, int GH, typename T, int NW, bool PAGED>
__global__ __launch_bounds__(NW * 64) void split_kernel(SplitArgs a) {
  using C = SplitCfg<D, GH, T, NW>;
  using V16 = typename KVT<T>::vec;
  constexpr int VW = C::VW, LPR = C::LPR, NV = C::NV, EPL = C::EPL, RPS = C::RPS;
  constexpr int LPR2 = C::LPR2, RPI = C::RPI, UQK = C::UQK, UPV = C::UPV;
  constexpr int NT = NW * 64;

  extern __shared__ float smem[];
  // layout: sc [chunk][GH] | red [NW][GH][D] | wstat [NW][GH] | blk [chunk/page + 2]
  float* sc = smem;
  float* red = sc + a.chunk * GH;
  float* wstat = red + NW * GH * D;
  int32_t* sblk = reinterpret_cast<int32_t*>(wstat + NW * GH);

  const int c = blockIdx.x;
  const int G = a.nq / a.nkv;
  const int nsub = G / GH;
  const int h = blockIdx.y / nsub;
  const int hq0 = h * G + (blockIdx.y % nsub) * GH;
  const int b = blockIdx.z;

  int n = a.n, t0 = a.t0;
  if constexpr (PAGED) {
    n = a.seq_lens[b];
    const int p = a.pos_arr ? a.pos_arr[b] : n - 1;
    t0 = (a.window > 0 && p - a.window + 1 > 0) ? p - a.window + 1 : 0;
    if (t0 > n) t0 = n;
  }
  const int tb = t0 + c * a.chunk;
  const int cnt = min(a.chunk, n - tb);
  if (cnt <= 0) return;  // whole workgroup: chunk past this sequence's end

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;

  const T* __restrict__ Kb = reinterpret_cast<const T*>(a.k);
  const T* __restrict__ Vb = reinterpret_cast<const T*>(a.v);
  int64_t hoff = (int64_t)h * a.head_stride;

  if constexpr (PAGED) {
    // block ids of this chunk, staged once
    const int p0 = tb >> a.page_shift;
    const int p1 = (tb + cnt - 1) >> a.page_shift;
    for (int i = tid; i <= p1 - p0; i += NT)
      sblk[i] = a.block_table[(int64_t)b * a.max_blocks + p0 + i];
    __syncthreads();
  }
  auto row_ptr = [&](const T* base, int t) -> const T* {
    if constexpr (PAGED) {
      const int pg = (t >> a.page_shift) - (tb >> a.page_shift);
      const int64_t blk = sblk[pg];
      return base + blk * a.block_stride + hoff +
             (int64_t)(t & ((1 << a.page_shift) - 1)) * a.tok_stride;
    } else {
      return base + (int64_t)t * a.tok_stride + hoff;
    }
  };

  // ---- pass 1: scores s[t][g] = (q_g . K_t) * scale ----
  const int s = lane % LPR;
  const int rr = lane / LPR;
  float qr[GH][EPL];
  {
    const float* qb = a.q + ((int64_t)b * a.nq + hq0) * D;
#pragma unroll
    for (int g = 0; g < GH; ++g)
#pragma unroll
      for (int v = 0; v < NV; ++v)
#pragma unroll
        for (int e4 = 0; e4 < VW; e4 += 4) {
          const f32x4 x = *reinterpret_cast<const f32x4*>(qb + g * D + (v * LPR + s) * VW + e4);
          qr[g][v * VW + e4 + 0] = x[0];
          qr[g][v * VW + e4 + 1] = x[1];
          qr[g][v * VW + e4 + 2] = x[2];
          qr[g][v * VW + e4 + 3] = x[3];
        }
  }
  float mloc[GH];
#pragma unroll
  for (int g = 0; g < GH; ++g) mloc[g] = -INFINITY;

  for (int r0 = w * RPS; r0 < cnt; r0 += NW * RPS * UQK) {
    V16 kv[UQK][NV];
#pragma unroll
    for (int u = 0; u < UQK; ++u) {
      const int row = r0 + u * NW * RPS + rr;
      if (row < cnt) {
        const T* p = row_ptr(Kb, tb + row);
#pragma unroll
        for (int v = 0; v < NV; ++v) kv[u][v] = load16(p + (v * LPR + s) * VW);
      } else {
#pragma unroll
        for (int v = 0; v < NV; ++v) kv[u][v] = V16{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int u = 0; u < UQK; ++u) {
      float acc[GH];
#pragma unroll
      for (int g = 0; g < GH; ++g) acc[g] = 0.f;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        float x[VW];
        KVT<T>::unpack(kv[u][v], x);
#pragma unroll
        for (int e = 0; e < VW; ++e)
#pragma unroll
          for (int g = 0; g < GH; ++g) acc[g] = fmaf(qr[g][v * VW + e], x[e], acc[g]);
      }
      const int row = r0 + u * NW * RPS + rr;
#pragma unroll
      for (int g = 0; g < GH; ++g) acc[g] = group_sum<LPR>(acc[g]) * a.scale;
      if (row < cnt) {
#pragma unroll
        for (int g = 0; g < GH; ++g) mloc[g] = fmaxf(mloc[g], acc[g]);
        if (s == 0) {
#pragma unroll
          for (int g = 0; g < GH; ++g) sc[row * GH + g] = acc[g];
        }
      }
    }
  }

  // ---- chunk max per head ----
#pragma unroll
  for (int g = 0; g < GH; ++g) {
    const float m = wave_max(mloc[g]);
    if (lane == 0) wstat[w * GH + g] = m;
  }
  __syncthreads();
  float M[GH];
#pragma unroll
  for (int g = 0; g < GH; ++g) {
    float m = wstat[g];
#pragma unroll
    for (int ww = 1; ww < NW; ++ww) m = fmaxf(m, wstat[ww * GH + g]);
    M[g] = m;
  }
  __syncthreads();  // wstat is reused for the sums below

  // ---- pass 2: p = exp(s - M), chunk sums ----
  // NT is a multiple of GH, so thread tid always handles head g = tid % GH.
  float lsum = 0.f;
  {
    const int g = tid % GH;
    float mg = M[0];
#pragma unroll
    for (int gg = 1; gg < GH; ++gg)
      if (g == gg) mg = M[gg];
    for (int idx = tid; idx < cnt * GH; idx += NT) {
      const float p = softmax_exp(sc[idx] - mg);
      sc[idx] = p;
      lsum += p;
    }
  }
#pragma unroll
  for (int off = GH; off < 64; off <<= 1) lsum += __shfl_xor(lsum, off);
  if (lane < GH) wstat[w * GH + lane] = lsum;
  __syncthreads();
  float L[GH];
#pragma unroll
  for (int g = 0; g < GH; ++g) {
    float l = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) l += wstat[ww * GH + g];
    L[g] = l;
  }

  // ---- pass 3: o_g = sum_t p[t][g] * V_t ----
  const int cs = lane % LPR2;
  const int rs = lane / LPR2;
  float acc[GH][VW];
#pragma unroll
  for (int g = 0; g < GH; ++g)
#pragma unroll
    for (int e = 0; e < VW; ++e) acc[g][e] = 0.f;

  for (int r0 = w * RPI; r0 < cnt; r0 += NW * RPI * UPV) {
    V16 vv[UPV];
    float pw[UPV][GH];
#pragma unroll
    for (int u = 0; u < UPV; ++u) {
      const int row = r0 + u * NW * RPI + rs;
      if (row < cnt) {
        vv[u] = load16(row_ptr(Vb, tb + row) + cs * VW);
#pragma unroll
        for (int g = 0; g < GH; ++g) pw[u][g] = sc[row * GH + g];
      } else {
        vv[u] = V16{0, 0, 0, 0};
#pragma unroll
        for (int g = 0; g < GH; ++g) pw[u][g] = 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < UPV; ++u) {
      float x[VW];
      KVT<T>::unpack(vv[u], x);
#pragma unroll
      for (int g = 0; g < GH; ++g)
#pragma unroll
        for (int e = 0; e < VW; ++e) acc[g][e] = fmaf(pw[u][g], x[e], acc[g][e]);
    }
  }
  // rows handled by different lane groups of the wave
#pragma unroll
  for (int off = LPR2; off < 64; off <<= 1)
#pragma unroll
    for (int g = 0; g < GH; ++g)
#pragma unroll
      for (int e = 0; e < VW; ++e) acc[g][e] += __shfl_xor(acc[g][e], off);
  if (rs == 0) {
#pragma unroll
    for (int g = 0; g < GH; ++g)
#pragma unroll
      for (int e = 0; e < VW; ++e) red[(w * GH + g) * D + cs * VW + e] = acc[g][e];
  }
  __syncthreads();

  const int64_t obase = (int64_t)b * a.nq + hq0;
  for (int idx = tid; idx < GH * D; idx += NT) {
    float sum = red[idx];
#pragma unroll
    for (int ww = 1; ww < NW; ++ww) sum += red[ww * GH * D + idx];
    const int g = idx / D;
    const int j = idx - g * D;
    if (a.direct) {
      float lg = L[0];
#pragma unroll
      for (int gg = 1; gg < GH; ++gg)
        if (g == gg) lg = L[gg];
      a.o[(obase + g) * D + j] = sum / lg;
    } else {
      a.part_o[((obase + g) * a.nchunks + c) * D + j] = sum;
    }
  }
  if (!a.direct && tid < GH) {
    float mg = M[0], lg = L[0];
#pragma unroll
    for (int gg = 1; gg < GH; ++gg)
      if (tid == gg) {
        mg = M[gg];
        lg = L[gg];
      }
    float* ml = a.part_ml + ((obase + tid) * a.nchunks + c) * 2;
    ml[0] = mg;
    ml[1] = lg;
  }
}

// ---------------------------------------------------------------------------
// Log-sum-exp combine: o = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c.
struct CombineArgs {
  const float* part_o;
  const float* part_ml;
  float* o;
  const int32_t* seq_lens;
  const int32_t* pos_arr;
  int nq, d, nchunks, chunk, n, t0, window;
};

template <bool PAGED>
__global__ __launch_bounds__(256) void combine_kernel(CombineArgs a) {
  extern __shared__ float wts[];  // [nchunks]
  __shared__ float red[8];
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  int nch = a.nchunks;
  if constexpr (PAGED) {
    const int n = a.seq_lens[b];
    const int p = a.pos_arr ? a.pos_arr[b] : n - 1;
    int t0 = (a.window > 0 && p - a.window + 1 > 0) ? p - a.window + 1 : 0;
    if (t0 > n) t0 = n;
    nch = (n - t0 + a.chunk - 1) / a.chunk;
    if (nch > a.nchunks) nch = a.nchunks;  // never past the partials written
  }
  const int64_t row = (int64_t)b * a.nq + hq;
  float* out = a.o + row * a.d;
  if (nch <= 0) {
    for (int j = tid; j < a.d; j += blockDim.x) out[j] = 0.f;
    return;
  }
  const float* ml = a.part_ml + row * a.nchunks * 2;
  const float* po = a.part_o + row * a.nchunks * a.d;

  float m = -INFINITY;
  for (int c = tid; c < nch; c += blockDim.x) m = fmaxf(m, ml[2 * c]);
  m = wave_max(m);
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  float M = red[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); ++i) M = fmaxf(M, red[i]);
  __syncthreads();

  float l = 0.f;
  for (int c = tid; c < nch; c += blockDim.x) {
    const float wgt = softmax_exp(ml[2 * c] - M);
    wts[c] = wgt;
    l += wgt * ml[2 * c + 1];
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) l += __shfl_xor(l, off);
  if ((tid & 63) == 0) red[tid >> 6] = l;
  __syncthreads();
  float L = 0.f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) L += red[i];
  const float inv = 1.0f / L;

  for (int j = tid; j < a.d; j += blockDim.x) {
    float acc = 0.f;
    for (int c = 0; c < nch; ++c) acc = fmaf(wts[c], po[(int64_t)c * a.d + j], acc);
    out[j] = acc * inv;
  }
}

__global__ void vexp_kernel(const float* x, float* y, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = softmax_exp(x[i]);
}

__global__ void zero_kernel(float* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

// ---------------------------------------------------------------------------
// Host side.

constexpr int kWaves = 4;  // waves per split workgroup
constexpr int kMaxChunk = 1024;
constexpr int kMaxScores = 4096;  // chunk * heads-per-workgroup (16 KB of LDS scores)

int g_split_chunk = 0;  // 0 = automatic

struct WsKey {
  int dev;
  void* stream;
  bool operator<(const WsKey& o) const {
    return dev != o.dev ? dev < o.dev : stream < o.stream;
  }
};
struct WsBuf {
  void* ptr = nullptr;
  size_t bytes = 0;
};
std::mutex g_ws_mu;
std::map<WsKey, WsBuf> g_ws;

// Per-(device, stream) workspace, grown on demand.  Growth waits for the
// stream so the old buffer is no longer in use when freed.
int workspace(void* stream, size_t bytes, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  std::lock_guard<std::mutex> lk(g_ws_mu);
  WsBuf& w = g_ws[WsKey{dev, stream}];
  if (w.bytes < bytes) {
    if (w.ptr) {
      e = hipStreamSynchronize((hipStream_t)stream);
      if (e != hipSuccess) return (int)e;
      e = hipFree(w.ptr);
      if (e != hipSuccess) return (int)e;
      w.ptr = nullptr;
      w.bytes = 0;
    }
    size_t want = bytes < (size_t)(4u << 20) ? (size_t)(4u << 20) : bytes;
    e = hipMalloc(&w.ptr, want);
    if (e != hipSuccess) return (int)e;
    w.bytes = want;
  }
  *out = w.ptr;
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

// Tokens per chunk: enough chunks that the launch holds ~8 workgroups per CU
// (several resident per CU, so HBM stays busy through the tail), rounded to
// 16 tokens.
int plan_chunk(int n_att, int rows_of_wgs, int gh) {
  int chunk = g_split_chunk;
  if (chunk <= 0) {
    const long target = 8L * num_cus();
    long nch = (target + rows_of_wgs - 1) / rows_of_wgs;
    if (nch < 1) nch = 1;
    chunk = (int)((n_att + nch - 1) / nch);
    chunk = (chunk + 15) & ~15;
    if (chunk < 64) chunk = 64;
  }
  if (chunk > kMaxChunk) chunk = kMaxChunk;
  if (chunk * gh > kMaxScores) chunk = kMaxScores / gh;
  if (chunk < 16) chunk = 16;
  return chunk;
}

template <int D, int GH, typename T, bool PAGED>
hipError_t launch_split(const SplitArgs& a, int nsubs, int B, hipStream_t st) {
  using C = SplitCfg<D, GH, T, kWaves>;
  (void)sizeof(C);
  const int max_pages = a.chunk + 2;  // pages one chunk can touch (page >= 1)
  size_t lds = sizeof(float) * ((size_t)a.chunk * GH + (size_t)kWaves * GH * D + kWaves * GH) +
               (PAGED ? sizeof(int32_t) * (size_t)max_pages : 0);
  if (lds > 65536) return hipErrorInvalidConfiguration;
  dim3 grid(a.nchunks, a.nkv * nsubs, B);
  hipLaunchKernelGGL((split_kernel<D, GH, T, kWaves, PAGED>), grid, dim3(kWaves * 64), lds, st,
                     a);
  return hipGetLastError();
}

template <int D, typename T, bool PAGED>
hipError_t dispatch_gh(int gh, const SplitArgs& a, int nsubs, int B, hipStream_t st) {
  switch (gh) {
    case 1: return launch_split<D, 1, T, PAGED>(a, nsubs, B, st);
    case 2: return launch_split<D, 2, T, PAGED>(a, nsubs, B, st);
    case 4: return launch_split<D, 4, T, PAGED>(a, nsubs, B, st);
    case 8: return launch_split<D, 8, T, PAGED>(a, nsubs, B, st);
  }
  return hipErrorInvalidValue;
}

template <bool PAGED>
hipError_t dispatch_split(int d, int kv_dtype, int gh, const SplitArgs& a, int nsubs, int B,
                          hipStream_t st) {
  if (kv_dtype == MOLOT_KV_F32) {
    switch (d) {
      case 64: return dispatch_gh<64, float, PAGED>(gh, a, nsubs, B, st);
      case 128: return dispatch_gh<128, float, PAGED>(gh, a, nsubs, B, st);
      case 256: return dispatch_gh<256, float, PAGED>(gh, a, nsubs, B, st);
    }
  } else {
    switch (d) {
      case 64: return dispatch_gh<64, bf16_t, PAGED>(gh, a, nsubs, B, st);
      case 128: return dispatch_gh<128, bf16_t, PAGED>(gh, a, nsubs, B, st);
      case 256: return dispatch_gh<256, bf16_t, PAGED>(gh, a, nsubs, B, st);
    }
  }
  return hipErrorInvalidValue;
}

bool supported_d(int d) { return d == 64 || d == 128 || d == 256; }

int check_common(int nq, int nkv, int d, int kv_dtype) {
  if (nq <= 0 || nkv <= 0 || nq % nkv != 0) return MOLOT_EINVAL;
  if (kv_dtype != MOLOT_KV_F32 && kv_dtype != MOLOT_KV_BF16) return MOLOT_EINVAL;
  if (!supported_d(d)) return MOLOT_ENOTSUP;
  return 0;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int zero_out(float* O, int64_t count, hipStream_t st) {
  if (count <= 0) return 0;
  const int64_t blocks = (count + 255) / 256;
  hipLaunchKernelGGL(zero_kernel, dim3((unsigned)blocks), dim3(256), 0, st, O, count);
  return (int)hipGetLastError();
}

}  // namespace

// ===========================================================================
// C ABI
extern "C" {

const char* molot_hip_strerror(int status) {
  switch (status) {
    case MOLOT_OK: return "ok";
    case MOLOT_EINVAL: return "molot_amd: invalid argument";
    case MOLOT_ENOTSUP: return "molot_amd: unsupported shape (head dim must be 64, 128 or 256)";
    case MOLOT_ENOSPC: return "molot_amd: KV cache full";
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "molot_amd: unknown status";
}

const char* molot_hip_version(void) { return "molot_amd 0.1"; }

void molot_rope_inv_freq(float base, int d, float* out) {
  for (int i = 0; i < d / 2; ++i) out[i] = 1.0f / powf(base, (2.0f * (float)i) / (float)d);
}

void molot_hip_set_split_chunk(int tokens) { g_split_chunk = tokens > 0 ? tokens : 0; }

int molot_hip_split_plan(int nkv, int n_att, int d, int kv_dtype, int* nchunks, int* chunk) {
  (void)d;
  (void)kv_dtype;
  if (nkv <= 0 || n_att < 0 || !nchunks || !chunk) return MOLOT_EINVAL;
  const int ch = plan_chunk(n_att, nkv, 4);
  *chunk = ch;
  *nchunks = (n_att + ch - 1) / ch;
  return 0;
}

int molot_hip_rope_apply(float* x, int nheads, int d, int pos, const float* inv_freq,
                         void* stream) {
  if (!x || !inv_freq || nheads < 0 || d <= 0 || (d & 1) || d > 2048) return MOLOT_EINVAL;
  if (nheads == 0) return 0;
  RopeArgs a{};
  a.q = x;
  a.inv_freq = inv_freq;
  a.nq = nheads;
  a.nkv = 0;
  a.d = d;
  a.pos = pos;
  a.append = 0;
  hipLaunchKernelGGL(rope_append_kernel, dim3(nheads, 1), dim3(((d / 2) + 63) / 64 * 64), 0,
                     (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

int molot_hip_rope_append(float* q, const float* k_new, const float* v_new, void* K, void* V,
                          int nq, int nkv, int d, int slot, int pos, const float* inv_freq,
                          int kv_dtype, void* stream) {
  if (nq < 0 || nkv <= 0 || d <= 0 || (d & 1) || d > 2048 || slot < 0) return MOLOT_EINVAL;
  if ((nq > 0 && !q) || !k_new || !v_new || !K || !V || !inv_freq) return MOLOT_EINVAL;
  if (kv_dtype != MOLOT_KV_F32 && kv_dtype != MOLOT_KV_BF16) return MOLOT_EINVAL;
  RopeArgs a{};
  a.q = q;
  a.k_new = k_new;
  a.v_new = v_new;
  a.K = K;
  a.V = V;
  a.inv_freq = inv_freq;
  a.tok_stride = (int64_t)nkv * d;
  a.head_stride = d;
  a.nq = nq;
  a.nkv = nkv;
  a.d = d;
  a.slot = slot;
  a.pos = pos;
  a.kv_dtype = kv_dtype;
  a.append = 1;
  hipLaunchKernelGGL(rope_append_kernel, dim3(nq + nkv, 1), dim3(((d / 2) + 63) / 64 * 64), 0,
                     (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

int molot_hip_attn_decode_strided(const float* Q, const void* K, const void* V, float* O, int nq,
                                  int nkv, int n, int d, int64_t tok_stride, int64_t head_stride,
                                  float scale, int pos_cur, int window, int kv_dtype,
                                  void* stream) {
  int st = check_common(nq, nkv, d, kv_dtype);
  if (st) return st;
  if (!Q || !O || n < 0) return MOLOT_EINVAL;
  hipStream_t hs = (hipStream_t)stream;
  int t0 = (window > 0 && pos_cur - window + 1 > 0) ? pos_cur - window + 1 : 0;
  if (t0 > n) t0 = n;
  const int n_att = n - t0;
  if (n_att <= 0) return zero_out(O, (int64_t)nq * d, hs);  // empty range: o = 0
  if (!K || !V) return MOLOT_EINVAL;
  const int esz = kv_dtype == MOLOT_KV_F32 ? 4 : 2;
  // 16-byte vector loads of every row
  if (!aligned16(K) || !aligned16(V) || !aligned16(Q) || (tok_stride * esz) % 16 ||
      (head_stride * esz) % 16)
    return MOLOT_EINVAL;
  const int G = nq / nkv;
  const int gh = pick_gh(G);
  const int nsubs = G / gh;
  SplitArgs a{};
  a.q = Q;
  a.k = K;
  a.v = V;
  a.o = O;
  a.tok_stride = tok_stride;
  a.head_stride = head_stride;
  a.nq = nq;
  a.nkv = nkv;
  a.n = n;
  a.t0 = t0;
  a.window = window;
  a.scale = scale;
  a.chunk = plan_chunk(n_att, nkv * nsubs, gh);
  a.nchunks = (n_att + a.chunk - 1) / a.chunk;
  a.direct = a.nchunks == 1;
  if (!a.direct) {
    const size_t po = (size_t)nq * a.nchunks * d;
    const size_t pml = (size_t)nq * a.nchunks * 2;
    void* ws = nullptr;
    st = workspace(stream, (po + pml) * sizeof(float), &ws);
    if (st) return st;
    a.part_o = (float*)ws;
    a.part_ml = a.part_o + po;
  }
  hipError_t e = dispatch_split<false>(d, kv_dtype, gh, a, nsubs, 1, hs);
  if (e != hipSuccess) return (int)e;
  if (a.direct) return 0;
  CombineArgs c{};
  c.part_o = a.part_o;
  c.part_ml = a.part_ml;
  c.o = O;
  c.nq = nq;
  c.d = d;
  c.nchunks = a.nchunks;
  c.chunk = a.chunk;
  hipLaunchKernelGGL(combine_kernel<false>, dim3(nq, 1), dim3(d >= 256 ? 256 : 128),
                     sizeof(float) * (size_t)a.nchunks, hs, c);
  return (int)hipGetLastError();
}

int molot_hip_attn_decode_gqa_cache(const float* Q, const void* K, const void* V, float* O,
                                    int nq, int nkv, int n, int qhd, float scale, int pos_cur,
                                    int window, int kv_dtype, void* stream) {
  return molot_hip_attn_decode_strided(Q, K, V, O, nq, nkv, n, qhd, (int64_t)nkv * qhd, qhd,
                                       scale, pos_cur, window, kv_dtype, stream);
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

int molot_hip_decode_step(float* q, const float* k_new, const float* v_new, void* K, void* V,
                          float* O, int nq, int nkv, int d, int slot, int pos,
                          const float* inv_freq, float scale, int window, int kv_dtype,
                          void* stream) {
  int st = check_common(nq, nkv, d, kv_dtype);
  if (st) return st;
  st = molot_hip_rope_append(q, k_new, v_new, K, V, nq, nkv, d, slot, pos, inv_freq, kv_dtype,
                             stream);
  if (st) return st;
  return molot_hip_attn_decode_gqa_cache(q, K, V, O, nq, nkv, slot + 1, d, scale, pos, window,
                                         kv_dtype, stream);
}

int molot_hip_attn_decode_paged(const float* Q, const void* K, const void* V, float* O,
                                const int32_t* block_table, const int32_t* seq_lens,
                                const int32_t* pos, int B, int max_blocks, int max_seq_len,
                                int nq, int nkv, int d, int page, float scale, int window,
                                int kv_dtype, void* stream) {
  int st = check_common(nq, nkv, d, kv_dtype);
  if (st) return st;
  if (!Q || !K || !V || !O || !block_table || !seq_lens || B < 0 || max_blocks <= 0 ||
      max_seq_len < 0 || page <= 0 || (page & (page - 1)))
    return MOLOT_EINVAL;
  if ((int64_t)max_seq_len > (int64_t)max_blocks * page) return MOLOT_EINVAL;
  if (!aligned16(K) || !aligned16(V) || !aligned16(Q)) return MOLOT_EINVAL;
  if (B == 0) return 0;
  hipStream_t hs = (hipStream_t)stream;
  int shift = 0;
  while ((1 << shift) < page) ++shift;
  const int G = nq / nkv;
  const int gh = pick_gh(G);
  const int nsubs = G / gh;
  SplitArgs a{};
  a.q = Q;
  a.k = K;
  a.v = V;
  a.o = O;
  a.block_table = block_table;
  a.seq_lens = seq_lens;
  a.pos_arr = pos;
  a.tok_stride = d;
  a.head_stride = (int64_t)page * d;
  a.block_stride = (int64_t)nkv * page * d;
  a.nq = nq;
  a.nkv = nkv;
  a.max_blocks = max_blocks;
  a.page_shift = shift;
  a.window = window;
  a.scale = scale;
  // widest attended range of any sequence: with pos[] given, pos may lag the
  // cache end, so only max_seq_len bounds it
  const int span = (!pos && window > 0 && window < max_seq_len) ? window : max_seq_len;
  a.chunk = plan_chunk(span > 0 ? span : 1, nkv * nsubs * B, gh);
  if (a.chunk % page) a.chunk = (a.chunk / page + 1) * page;
  while (a.chunk > page && (a.chunk > kMaxChunk || a.chunk * gh > kMaxScores)) a.chunk -= page;
  a.nchunks = (span + a.chunk - 1) / a.chunk;
  if (a.nchunks < 1) a.nchunks = 1;
  a.direct = 0;
  const size_t po = (size_t)B * nq * a.nchunks * d;
  const size_t pml = (size_t)B * nq * a.nchunks * 2;
  void* ws = nullptr;
  st = workspace(stream, (po + pml) * sizeof(float), &ws);
  if (st) return st;
  a.part_o = (float*)ws;
  a.part_ml = a.part_o + po;
  hipError_t e = dispatch_split<true>(d, kv_dtype, gh, a, nsubs, B, hs);
  if (e != hipSuccess) return (int)e;
  CombineArgs c{};
  c.part_o = a.part_o;
  c.part_ml = a.part_ml;
  c.o = O;
  c.seq_lens = seq_lens;
  c.pos_arr = pos;
  c.nq = nq;
  c.d = d;
  c.nchunks = a.nchunks;
  c.chunk = a.chunk;
  c.window = window;
  hipLaunchKernelGGL(combine_kernel<true>, dim3(nq, B), dim3(d >= 256 ? 256 : 128),
                     sizeof(float) * (size_t)a.nchunks, hs, c);
  return (int)hipGetLastError();
}

int molot_hip_rope_append_paged(float* q, const float* k_new, const float* v_new, void* K,
                                void* V, const int32_t* block_table, const int32_t* seq_lens,
                                const int32_t* pos, int B, int max_blocks, int nq, int nkv, int d,
                                int page, const float* inv_freq, int kv_dtype, void* stream) {
  if (nq < 0 || nkv <= 0 || d <= 0 || (d & 1) || d > 2048 || B < 0 || max_blocks <= 0 ||
      page <= 0)
    return MOLOT_EINVAL;
  if ((nq > 0 && !q) || !k_new || !v_new || !K || !V || !inv_freq || !block_table || !seq_lens)
    return MOLOT_EINVAL;
  if (kv_dtype != MOLOT_KV_F32 && kv_dtype != MOLOT_KV_BF16) return MOLOT_EINVAL;
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
  a.tok_stride = d;
  a.head_stride = (int64_t)page * d;
  a.block_stride = (int64_t)nkv * page * d;
  a.nq = nq;
  a.nkv = nkv;
  a.d = d;
  a.max_blocks = max_blocks;
  a.page = page;
  a.kv_dtype = kv_dtype;
  a.append = 1;
  hipLaunchKernelGGL(rope_append_kernel, dim3(nq + nkv, B), dim3(((d / 2) + 63) / 64 * 64), 0,
                     (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

int molot_hip_vexp(const float* x, float* y, int64_t n, void* stream) {
  if (n < 0 || (n > 0 && (!x || !y))) return MOLOT_EINVAL;
  if (n == 0) return 0;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(vexp_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, x,
                     y, n);
  return (int)hipGetLastError();
}

}  // extern "C"
