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

// K/V rows are read exactly once per step: non-temporal 16-byte loads (the
// streaming hint measurably raises the sustained HBM read rate on gfx950).
template <typename T>
__device__ __forceinline__ typename KVT<T>::vec load16(const T* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const typename KVT<T>::vec*>(p));
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

// Cross-workgroup hand-off of the split-K partials.  The L2 of each XCD is
// not coherent with the others, and an agent-scope fence writes back and
// invalidates a whole L2, which would disturb every workgroup streaming KV
// through it.  The partials therefore travel per access at device scope:
// stores are written through to the device coherence point (sc1), each
// thread waits for its stores to complete before the workgroup's counter
// increment (a device-coherent atomic), and the finishing workgroup reads
// them back with device-scope loads (sc1), which do not hit stale lines.
__device__ __forceinline__ void store_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_dev(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
// Fused decode attention.
//
// Grid (chunks, nkv * subgroups, sequences).  Workgroup (c, h/sub, b) owns the
// context rows [tb, tb + cnt) of KV head h and the GH query heads
// hq0 .. hq0+GH-1 of that head's group:
//   1. prologue: q of the GH heads into LDS; with ROPE, rotated there, and the
//      workgroup holding the chunk that contains the new token rotates k_new,
//      rounds k/v to the cache type, keeps them in LDS and (subgroup 0)
//      stores them into the cache slot n-1;
//   2. every wave streams its blocks of RB rows: 16-byte loads of the block's
//      K and V rows are issued together; scores of the GH heads per K row
//      (LPR lanes per row, DPP sums); online softmax per wave (running max,
//      rescale of the accumulators); probabilities through a per-wave LDS
//      slice to the PV lanes (LPR2 lanes per V row, 16 bytes each);
//   3. the new token (ROPE, last chunk) is folded in by wave 0 from LDS;
//   4. the waves' (max, sum, o) are merged through LDS; a single-chunk
//      problem writes o / sum directly, otherwise the chunk partial goes to
//      the workspace and the workgroup that finishes a head group last (a
//      self-resetting counter) merges all chunk partials of that group with
//      log-sum-exp weights, writes O and, with ROPE, the rotated q.
struct AttnArgs {
  const float* q;        // [B][nq][D]; un-rotated when the kernel applies RoPE
  float* q_out;          // [B][nq][D] rotated q (ROPE), written by the finishing workgroup
  const float* k_new;    // [B][nkv][D] fp32 (ROPE)
  const float* v_new;    // [B][nkv][D] fp32 (ROPE)
  void* k;               // KV cache
  void* v;
  const float* inv_freq; // [D/2] (ROPE)
  float* o;              // [B][nq][D]
  float* part_o;         // [B][nq][nchunks][D]
  float* part_ml;        // [B][nq][nchunks][2] = (max, sum)
  int* counters;         // [B][nkv * subgroups], zero between launches
  const int32_t* block_table;
  const int32_t* seq_lens;
  const int32_t* pos_arr;
  int64_t tok_stride, head_stride, block_stride;
  int nq, nkv, n, t0, pos, chunk, nchunks, max_blocks, page_shift, window;
  float scale;
};

// Work mapping of one kernel instance.
//   LPR  lanes cooperating on one K row in the score loop (DPP sums across them)
//   RB   rows per wave block (the block's K and V loads are issued together)
//   NW   waves per workgroup
template <int D, int GH, typename T, int LPR_, int RB_, int NW_>
struct Cfg {
  static constexpr int VW = KVT<T>::VW;
  static constexpr int LPR = LPR_;
  static constexpr int NV = D / (LPR * VW);  // 16-byte vectors per lane per K row
  static constexpr int EPL = NV * VW;        // q elements per lane
  static constexpr int RPS = 64 / LPR;       // K rows per wave step
  static constexpr int LPR2 = D / VW;        // lanes per V row (PV)
  static constexpr int RPI = 64 / LPR2;      // V rows per wave step
  static constexpr int RB = RB_;
  static constexpr int KS = RB / RPS;  // K steps per block
  static constexpr int VS = RB / RPI;  // V steps per block
  static constexpr int NW = NW_;
  static constexpr int NT = NW * 64;
  static_assert(NV >= 1 && D % (LPR * VW) == 0, "bad score mapping");
  static_assert(LPR2 <= 64 && 64 % LPR2 == 0, "bad PV mapping");
  static_assert(RB % RPS == 0 && RB % RPI == 0, "bad block");
};

// Default mapping: q registers (GH x D/LPR) kept at <= 32 where the 16-byte
// vector allows it, then the largest block (<= 16 loads in flight per lane)
// whose estimated register need keeps 4 waves per SIMD, else 2; 16 waves per
// workgroup when the wave-merge buffer (NW*GH*D floats) and 4 waves/SIMD
// allow, else 8 or 4.
template <int D, int GH, typename T>
struct Tune {
  static constexpr int VW = KVT<T>::VW;
  static constexpr int lpr() {
    int l = 8;
    while (GH * D / l > 32 && l < D / VW) l *= 2;
    return l;
  }
  static constexpr int LPR = lpr();
  static constexpr int NV = D / (LPR * VW);
  static constexpr int RPS = 64 / LPR, RPI = 64 / (D / VW);
  static constexpr int loads(int rb) { return (rb / RPS) * NV + rb / RPI; }
  static constexpr int regs(int rb) {
    return GH * NV * VW + GH * VW + 4 * loads(rb) + (rb / RPS) * GH + 3 * GH + 28;
  }
  static constexpr bool ok(int rb, int cap) {
    return rb % RPS == 0 && rb % RPI == 0 && loads(rb) <= 16 && regs(rb) <= cap;
  }
  static constexpr int rb() {
    for (int cap : {128, 232})
      for (int r : {32, 16, 8})
        if (ok(r, cap)) return r;
    return RPS > RPI ? RPS : RPI;
  }
  static constexpr int RB = rb();
  static constexpr int nw() {
    if (regs(RB) <= 128 && GH * D <= 512) return 16;
    return GH * D <= 1024 ? 8 : 4;
  }
  static constexpr int NW = nw();
  using C = Cfg<D, GH, T, LPR, RB, NW>;
};

// Dynamic LDS layout shared by host (size) and device (offsets), in floats.
struct Lds {
  int qs, cs, sn, knew, vnew, pw, wm, wl, wst, red, blk, flag, total;
  __host__ __device__ Lds(int D, int GH, int NW, int RB, int nchunks, int chunk, int page_shift,
                          bool paged) {
    int o = 0;
    qs = o; o += GH * D;
    cs = o; o += D / 2;
    sn = o; o += D / 2;
    knew = o; o += D;
    vnew = o; o += D;
    pw = o; o += NW * RB * GH;
    wm = o; o += NW * GH;
    wl = o; o += NW * GH;
    wst = o; o += 2 * NW * GH + 2 * GH;  // wave weights + (M, L); later the combine's phase stats
    red = o; o += NW * GH * D;
    blk = o; o += paged ? ((chunk >> page_shift) + 2) : 0;
    flag = o; o += 4;
    total = o;
  }
};

template <int D, int GH, typename T, bool PAGED, bool ROPE, typename C>
__global__ __launch_bounds__(C::NT) void attn_kernel(AttnArgs a) {
  using V16 = typename KVT<T>::vec;
  constexpr int VW = C::VW, LPR = C::LPR, NV = C::NV, EPL = C::EPL, RPS = C::RPS;
  constexpr int LPR2 = C::LPR2, RPI = C::RPI, RB = C::RB, KS = C::KS, VS = C::VS;
  constexpr int NW = C::NW, NT = C::NT;

  extern __shared__ float smem[];
  const Lds L(D, GH, NW, RB, a.nchunks, a.chunk, a.page_shift, PAGED);
  float* qs = smem + L.qs;
  float* knew = smem + L.knew;
  float* vnew = smem + L.vnew;

  const int c = blockIdx.x;
  const int G = a.nq / a.nkv;
  const int nsub = G / GH;
  const int sub = blockIdx.y % nsub;
  const int h = blockIdx.y / nsub;
  const int hq0 = h * G + sub * GH;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;

  int n = a.n, t0 = a.t0, pos = a.pos;
  if constexpr (PAGED) {
    n = a.seq_lens[b];
    pos = a.pos_arr ? a.pos_arr[b] : n - 1;
    t0 = (a.window > 0 && pos - a.window + 1 > 0) ? pos - a.window + 1 : 0;
    if (t0 > n) t0 = n;
  }
  // Chunks tile the cache rows [t0, cend); with ROPE the new token (slot
  // n-1) is not read from the cache but folded into the last chunk.
  const int cend = ROPE ? n - 1 : n;
  int nch = a.nchunks;
  if constexpr (PAGED) {
    const int span = cend - t0;
    nch = span > 0 ? (span + a.chunk - 1) / a.chunk : (ROPE ? 1 : 0);
    if (nch > a.nchunks) nch = a.nchunks;
  }
  if (c >= nch) {  // whole workgroup: chunk past this sequence's end
    if (c == 0)    // empty attended range: o = 0 (include/molot/attn.h:162 with no rows)
      for (int i = tid; i < GH * D; i += NT) a.o[((int64_t)b * a.nq + hq0) * D + i] = 0.f;
    return;
  }
  const int tb = t0 + c * a.chunk;
  const int cntg = max(0, min(a.chunk, cend - tb));  // rows read from the cache
  const bool is_new = ROPE && c == nch - 1;          // this chunk folds in the new token

  const T* __restrict__ Kb = reinterpret_cast<const T*>(a.k);
  const T* __restrict__ Vb = reinterpret_cast<const T*>(a.v);
  const int64_t hoff = (int64_t)h * a.head_stride;
  const int64_t qrow0 = (int64_t)b * a.nq + hq0;

  // ---- 1. prologue: block ids, the first block's loads, q (+ RoPE) ----
  if constexpr (PAGED) {
    int32_t* sblk_w = reinterpret_cast<int32_t*>(smem + L.blk);
    const int p0 = tb >> a.page_shift;
    const int p1 = (tb + cntg - 1) >> a.page_shift;
    for (int i = tid; cntg > 0 && i <= p1 - p0; i += NT)
      sblk_w[i] = a.block_table[(int64_t)b * a.max_blocks + p0 + i];
    __syncthreads();
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
  const int s = lane % LPR;    // scores: lane within a K row group
  const int rr = lane / LPR;   // scores: row of the group within a K step
  const int cs = lane % LPR2;  // PV: columns cs*VW .. cs*VW+VW-1
  const int rs = lane / LPR2;  // PV: row within a V step
  V16 kr[KS][NV];
  V16 vr[VS];
  auto load_block = [&](int rbase) {
#pragma unroll
    for (int k = 0; k < KS; ++k) {
      const int row = rbase + k * RPS + rr;
      if (row < cntg) {
        const T* p = row_ptr(Kb, tb + row);
#pragma unroll
        for (int v = 0; v < NV; ++v) kr[k][v] = load16(p + (v * LPR + s) * VW);
      } else {
#pragma unroll
        for (int v = 0; v < NV; ++v) kr[k][v] = V16{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int k = 0; k < VS; ++k) {
      const int row = rbase + k * RPI + rs;
      vr[k] = row < cntg ? load16(row_ptr(Vb, tb + row) + cs * VW) : V16{0, 0, 0, 0};
    }
  };
  const int nblk = (cntg + RB - 1) / RB;
  // The prologue's own global loads go first: loads retire in order, so
  // waiting for them does not also wait for the K/V block issued next.
  constexpr int QV = GH * D / 4;  // float4s of q of the group
  constexpr int QPT = (QV + NT - 1) / NT;
  static_assert(D <= NT, "one thread per head-dim element in the prologue");
  f32x4 qv[QPT];
#pragma unroll
  for (int u = 0; u < QPT; ++u) {
    const int i = tid + u * NT;
    if (i < QV) qv[u] = reinterpret_cast<const f32x4*>(a.q + qrow0 * D)[i];
  }
  float invf = 0.f, knv = 0.f, vnv = 0.f;
  if constexpr (ROPE) {
    if (tid < D / 2) invf = a.inv_freq[tid];
    if (is_new && tid < D) {
      knv = a.k_new[((int64_t)b * a.nkv + h) * D + tid];
      vnv = a.v_new[((int64_t)b * a.nkv + h) * D + tid];
    }
  }
  if (w < nblk) load_block(w * RB);  // in flight during the rest of the prologue
#pragma unroll
  for (int u = 0; u < QPT; ++u) {
    const int i = tid + u * NT;
    if (i < QV) reinterpret_cast<f32x4*>(qs)[i] = qv[u];
  }
  if constexpr (ROPE) {
    float* cs = smem + L.cs;
    float* sn = smem + L.sn;
    if (tid < D / 2) {
      const float ang = (float)pos * invf;
      double sd, cd;
      sincos((double)ang, &sd, &cd);
      cs[tid] = (float)cd;
      sn[tid] = (float)sd;
    }
    if (is_new && tid < D) {
      knew[tid] = knv;
      vnew[tid] = vnv;
    }
    __syncthreads();
    for (int i = tid; i < GH * (D / 2); i += NT) {
      const int g = i / (D / 2), j = i - g * (D / 2);
      const float x0 = qs[g * D + j], x1 = qs[g * D + j + D / 2];
      qs[g * D + j] = x0 * cs[j] - x1 * sn[j];
      qs[g * D + j + D / 2] = x0 * sn[j] + x1 * cs[j];
    }
    if (is_new) {
      // the appended row as the cache will hold it: rotated k, k and v in the cache type
      int64_t off;
      const int slot = n - 1;
      if constexpr (PAGED) {
        const int64_t blk = a.block_table[(int64_t)b * a.max_blocks + (slot >> a.page_shift)];
        off = blk * a.block_stride + hoff +
              (int64_t)(slot & ((1 << a.page_shift) - 1)) * a.tok_stride;
      } else {
        off = (int64_t)slot * a.tok_stride + hoff;
      }
      for (int j = tid; j < D / 2; j += NT) {
        const float k0 = knew[j], k1 = knew[j + D / 2];
        float r0 = k0 * cs[j] - k1 * sn[j];
        float r1 = k0 * sn[j] + k1 * cs[j];
        float v0 = vnew[j], v1 = vnew[j + D / 2];
        if constexpr (sizeof(T) == 2) {
          const uint16_t br0 = f32_to_bf16(r0), br1 = f32_to_bf16(r1);
          const uint16_t bv0 = f32_to_bf16(v0), bv1 = f32_to_bf16(v1);
          if (sub == 0) {
            uint16_t* kd = reinterpret_cast<uint16_t*>(a.k) + off;
            uint16_t* vd = reinterpret_cast<uint16_t*>(a.v) + off;
            kd[j] = br0;
            kd[j + D / 2] = br1;
            vd[j] = bv0;
            vd[j + D / 2] = bv1;
          }
          r0 = __uint_as_float((uint32_t)br0 << 16);
          r1 = __uint_as_float((uint32_t)br1 << 16);
          v0 = __uint_as_float((uint32_t)bv0 << 16);
          v1 = __uint_as_float((uint32_t)bv1 << 16);
        } else {
          if (sub == 0) {
            float* kd = reinterpret_cast<float*>(a.k) + off;
            float* vd = reinterpret_cast<float*>(a.v) + off;
            kd[j] = r0;
            kd[j + D / 2] = r1;
            vd[j] = v0;
            vd[j + D / 2] = v1;
          }
        }
        knew[j] = r0;
        knew[j + D / 2] = r1;
        vnew[j] = v0;
        vnew[j + D / 2] = v1;
      }
    }
  }
  __syncthreads();

  // q registers: lane s of a K row group holds elements (v*LPR + s)*VW + e
  float qr[GH][EPL];
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
  float m_run[GH], l_run[GH], acc[GH][VW];
#pragma unroll
  for (int g = 0; g < GH; ++g) {
    m_run[g] = -INFINITY;
    l_run[g] = 0.f;
#pragma unroll
    for (int e = 0; e < VW; ++e) acc[g][e] = 0.f;
  }

  for (int blk = w; blk < nblk; blk += NW) {
    const int rbase = blk * RB;
    if (blk != w) load_block(rbase);
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
      const bool valid = rbase + k * RPS + rr < cntg;
#pragma unroll
      for (int g = 0; g < GH; ++g) {
        const float t = group_sum<LPR>(d[g]) * a.scale;
        sc[k][g] = valid ? t : -INFINITY;
        bmax[g] = fmaxf(bmax[g], sc[k][g]);
      }
    }
    // block max across the wave's row groups, then the online update
#pragma unroll
    for (int g = 0; g < GH; ++g) {
#pragma unroll
      for (int off = LPR; off < 64; off <<= 1) bmax[g] = fmaxf(bmax[g], __shfl_xor(bmax[g], off));
      const float mn = fmaxf(m_run[g], bmax[g]);
      const float alpha = softmax_exp(m_run[g] - mn);  // m_run = -inf -> 0
      m_run[g] = mn;
      l_run[g] *= alpha;
#pragma unroll
      for (int e = 0; e < VW; ++e) acc[g][e] *= alpha;
    }
#pragma unroll
    for (int k = 0; k < KS; ++k) {
      if (s == 0) {
#pragma unroll
        for (int g = 0; g < GH; ++g) pw[(k * RPS + rr) * GH + g] = softmax_exp(sc[k][g] - m_run[g]);
      }
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int k = 0; k < VS; ++k) {
      float x[VW];
      KVT<T>::unpack(vr[k], x);
      float p[GH];
#pragma unroll
      for (int g = 0; g < GH; ++g) p[g] = pw[(k * RPI + rs) * GH + g];
#pragma unroll
      for (int g = 0; g < GH; ++g) {
        l_run[g] += p[g];
#pragma unroll
        for (int e = 0; e < VW; ++e) acc[g][e] = fmaf(p[g], x[e], acc[g][e]);
      }
    }
    __builtin_amdgcn_wave_barrier();
  }

  // ---- 3. the new token, from LDS ----
  if (is_new && w == 0) {
#pragma unroll
    for (int g = 0; g < GH; ++g) {
      float part = 0.f;
#pragma unroll
      for (int j = lane; j < D; j += 64) part = fmaf(qs[g * D + j], knew[j], part);
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) part += __shfl_xor(part, off);
      const float snew = part * a.scale;
      const float mn = fmaxf(m_run[g], snew);
      const float alpha = softmax_exp(m_run[g] - mn);
      const float p = softmax_exp(snew - mn);
      m_run[g] = mn;
      l_run[g] = l_run[g] * alpha + (rs == 0 ? p : 0.f);
#pragma unroll
      for (int e = 0; e < VW; ++e)
        acc[g][e] = acc[g][e] * alpha + (rs == 0 ? p * vnew[cs * VW + e] : 0.f);
    }
  }

  // ---- 4. merge the waves ----
#pragma unroll
  for (int off = LPR2; off < 64; off <<= 1)
#pragma unroll
    for (int g = 0; g < GH; ++g) {
      l_run[g] += __shfl_xor(l_run[g], off);
#pragma unroll
      for (int e = 0; e < VW; ++e) acc[g][e] += __shfl_xor(acc[g][e], off);
    }
  float* wm = smem + L.wm;
  float* wl = smem + L.wl;
  float* red = smem + L.red;
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < GH; ++g) {
      wm[w * GH + g] = m_run[g];
      wl[w * GH + g] = l_run[g];
    }
  }
  if (rs == 0) {
#pragma unroll
    for (int g = 0; g < GH; ++g)
#pragma unroll
      for (int e = 0; e < VW; ++e) red[(w * GH + g) * D + cs * VW + e] = acc[g][e];
  }
  __syncthreads();
  // chunk statistics per head: wave weights e^(m_w - M), chunk max M, sum L
  float* wst = smem + L.wst;  // [GH][NW] weights | [GH] M | [GH] L
  if (tid < GH) {
    const int g = tid;
    float m = wm[g];
#pragma unroll
    for (int ww = 1; ww < NW; ++ww) m = fmaxf(m, wm[ww * GH + g]);
    float l = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      const float wgt = softmax_exp(wm[ww * GH + g] - m);  // waves without rows: e^-inf = 0
      wst[g * NW + ww] = wgt;
      l = fmaf(wgt, wl[ww * GH + g], l);
    }
    wst[GH * NW + g] = m;
    wst[GH * NW + GH + g] = l;
  }
  __syncthreads();
  const bool direct = nch == 1;
  for (int idx = tid; idx < GH * D; idx += NT) {
    const int g = idx / D;
    float o = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) o = fmaf(wst[g * NW + ww], red[ww * GH * D + idx], o);
    if (direct)
      a.o[qrow0 * D + idx] = o / wst[GH * NW + GH + g];
    else
      store_dev(a.part_o + ((qrow0 + g) * a.nchunks + c) * D + (idx - g * D), o);
  }
  if (direct) {
    if constexpr (ROPE) {
      if (a.q_out)
        for (int i = tid; i < GH * D; i += NT) a.q_out[qrow0 * D + i] = qs[i];
    }
    return;
  }
  if (tid < GH) {
    float* ml = a.part_ml + ((qrow0 + tid) * a.nchunks + c) * 2;
    store_dev(ml, wst[GH * NW + tid]);
    store_dev(ml + 1, wst[GH * NW + GH + tid]);
  }

  // ---- 5. the workgroup finishing this head group merges all chunks ----
  int* flag = reinterpret_cast<int*>(smem + L.flag);
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have completed
  __syncthreads();
  if (tid == 0) {
    int* ctr = a.counters + (int64_t)b * gridDim.y + blockIdx.y;
    const int done = atomicAdd(ctr, 1);
    const bool last = done == nch - 1;
    if (last) atomicExch(ctr, 0);  // ready for the next launch
    flag[0] = last;
  }
  __syncthreads();
  if (!flag[0]) return;

  // Thread t owns output (g, j) of phase ph and merges chunks c = ph (mod PH)
  // with its own running max: m, l and o of those chunks are loaded together
  // (one round trip), then the PH phase results are merged through LDS.
  constexpr int P = GH * D;
  constexpr int PH = NT >= P ? (NT / P < NW ? NT / P : NW) : 1;  // PH*P <= NW*GH*D floats
  float* pst = wst;  // [PH][GH][2] phase (max, sum); PH <= NW, wst holds 2*NW*GH + 2*GH floats
  for (int t = tid; t < PH * P; t += NT) {
    const int pair = t % P, ph = t / P;
    const int g = pair / D, j = pair - g * D;
    const float* src = a.part_o + (qrow0 + g) * a.nchunks * D + j;
    const float* mls = a.part_ml + (qrow0 + g) * a.nchunks * 2;
    float m = -INFINITY, acc = 0.f, lsum = 0.f;
    for (int c0 = ph; c0 < nch; c0 += 8 * PH) {
      float mv[8], lv[8], ov[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int cc = c0 + u * PH;
        const bool ok = cc < nch;
        mv[u] = ok ? load_dev(mls + 2 * cc) : -INFINITY;
        lv[u] = ok ? load_dev(mls + 2 * cc + 1) : 0.f;
        ov[u] = ok ? load_dev(src + (int64_t)cc * D) : 0.f;
      }
      float mn = m;
#pragma unroll
      for (int u = 0; u < 8; ++u) mn = fmaxf(mn, mv[u]);
      const float alpha = softmax_exp(m - mn);  // m = -inf on the first pass -> 0
      acc *= alpha;
      lsum *= alpha;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float wgt = softmax_exp(mv[u] - mn);  // absent chunks: e^-inf = 0
        acc = fmaf(wgt, ov[u], acc);
        lsum = fmaf(wgt, lv[u], lsum);
      }
      m = mn;
    }
    red[ph * P + pair] = acc;
    if (j == 0) {
      pst[(ph * GH + g) * 2] = m;
      pst[(ph * GH + g) * 2 + 1] = lsum;
    }
  }
  __syncthreads();
  for (int pair = tid; pair < P; pair += NT) {
    const int g = pair / D;
    float M = pst[g * 2];
#pragma unroll
    for (int ph = 1; ph < PH; ++ph) M = fmaxf(M, pst[(ph * GH + g) * 2]);
    float o = 0.f, l = 0.f;
#pragma unroll
    for (int ph = 0; ph < PH; ++ph) {
      const float wgt = softmax_exp(pst[(ph * GH + g) * 2] - M);  // phases without chunks: 0
      o = fmaf(wgt, red[ph * P + pair], o);
      l = fmaf(wgt, pst[(ph * GH + g) * 2 + 1], l);
    }
    a.o[qrow0 * D + pair] = o / l;
  }
  if constexpr (ROPE) {
    if (a.q_out)
      for (int i = tid; i < GH * D; i += NT) a.q_out[qrow0 * D + i] = qs[i];
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

constexpr int kMaxChunk = 2048;
constexpr int kMaxCounters = 1 << 16;  // (sequence, head group) pairs per launch
constexpr size_t kCounterBytes = sizeof(int) * kMaxCounters;

int g_split_chunk = 0;  // tokens per chunk, 0 = automatic
int g_wgs_per_cu = 0;   // workgroups per CU, 0 = the variant's default
int g_variant = 0;      // mapping variant of the 32q/8kv/d128 fp32 kernels (tuning sweeps)

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

// Per-(device, stream) workspace, grown on demand: [counters | partials].
// The counters sit at offset 0 of every workspace, are zeroed once when it
// is allocated and are left at zero by every launch (the finishing
// workgroup resets its counter).  Growth waits for the stream so the old
// buffer is idle when freed.
int workspace(void* stream, size_t bytes, int** counters, float** partials) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  std::lock_guard<std::mutex> lk(g_ws_mu);
  WsBuf& w = g_ws[WsKey{dev, stream}];
  const size_t need = kCounterBytes + bytes;
  if (w.bytes < need) {
    if (w.ptr) {
      e = hipStreamSynchronize((hipStream_t)stream);
      if (e != hipSuccess) return (int)e;
      e = hipFree(w.ptr);
      if (e != hipSuccess) return (int)e;
      w.ptr = nullptr;
      w.bytes = 0;
    }
    const size_t want = need < (size_t)(8u << 20) ? (size_t)(8u << 20) : need;
    e = hipMalloc(&w.ptr, want);
    if (e != hipSuccess) return (int)e;
    e = hipMemset(w.ptr, 0, kCounterBytes);
    if (e != hipSuccess) return (int)e;
    w.bytes = want;
  }
  *counters = reinterpret_cast<int*>(w.ptr);
  *partials = reinterpret_cast<float*>(reinterpret_cast<char*>(w.ptr) + kCounterBytes);
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
// per CU (all resident at once by default: 16 waves per CU), rounded up to a
// multiple of `align` (= waves x rows per block) so every wave of a
// workgroup gets the same number of blocks.
int plan_chunk(int span, int rows_of_wgs, int align, int wpc) {
  int chunk = g_split_chunk;
  if (chunk <= 0) {
    const long target = (long)(g_wgs_per_cu > 0 ? g_wgs_per_cu : wpc) * num_cus();
    long nch = (target + rows_of_wgs - 1) / rows_of_wgs;
    if (nch < 1) nch = 1;
    chunk = (int)((span + nch - 1) / nch);
    chunk = (chunk + align - 1) / align * align;
  }
  if (chunk > kMaxChunk) chunk = kMaxChunk;
  if (chunk < 8) chunk = 8;
  return chunk;
}

int plan_launch(AttnArgs& a, int d, int span, int gh, int nsubs, int B, bool paged, int align,
                int wpc, void* stream);

template <int D, int GH, typename T, bool PAGED, bool ROPE, typename C>
int launch_cfg(AttnArgs a, int span, int nsubs, int B, void* stream) {
  int st = plan_launch(a, D, span, GH, nsubs, B, PAGED, C::NW * C::RB,
                       C::NW >= 16 ? 1 : 16 / C::NW, stream);
  if (st) return st;
  const Lds L(D, GH, C::NW, C::RB, a.nchunks, a.chunk, a.page_shift, PAGED);
  const size_t lds = sizeof(float) * (size_t)L.total;
  if (lds > 65536) return (int)hipErrorInvalidConfiguration;
  dim3 grid(a.nchunks, a.nkv * nsubs, B);
  hipLaunchKernelGGL((attn_kernel<D, GH, T, PAGED, ROPE, C>), grid, dim3(C::NT), lds,
                     (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

template <int D, int GH, typename T, bool PAGED, bool ROPE>
int launch_attn(const AttnArgs& a, int span, int nsubs, int B, void* stream) {
  if constexpr (D == 128 && GH == 4 && sizeof(T) == 4 && !PAGED) {
    switch (g_variant) {  // alternative mappings of the headline shape, for sweeps
      case 1: return launch_cfg<D, GH, T, PAGED, ROPE, Cfg<D, GH, T, 16, 8, 8>>(a, span, nsubs, B, stream);
      case 2: return launch_cfg<D, GH, T, PAGED, ROPE, Cfg<D, GH, T, 16, 16, 8>>(a, span, nsubs, B, stream);
      case 3: return launch_cfg<D, GH, T, PAGED, ROPE, Cfg<D, GH, T, 8, 16, 8>>(a, span, nsubs, B, stream);
      default: break;
    }
  }
  return launch_cfg<D, GH, T, PAGED, ROPE, typename Tune<D, GH, T>::C>(a, span, nsubs, B, stream);
}

template <int D, typename T, bool PAGED, bool ROPE>
int dispatch_gh(int gh, const AttnArgs& a, int span, int nsubs, int B, void* st) {
  switch (gh) {
    case 1: return launch_attn<D, 1, T, PAGED, ROPE>(a, span, nsubs, B, st);
    case 2: return launch_attn<D, 2, T, PAGED, ROPE>(a, span, nsubs, B, st);
    case 4: return launch_attn<D, 4, T, PAGED, ROPE>(a, span, nsubs, B, st);
    case 8: return launch_attn<D, 8, T, PAGED, ROPE>(a, span, nsubs, B, st);
  }
  return MOLOT_EINVAL;
}

template <bool PAGED, bool ROPE>
int dispatch_attn(int d, int kv_dtype, int gh, const AttnArgs& a, int span, int nsubs, int B,
                  void* st) {
  if (kv_dtype == MOLOT_KV_F32) {
    switch (d) {
      case 64: return dispatch_gh<64, float, PAGED, ROPE>(gh, a, span, nsubs, B, st);
      case 128: return dispatch_gh<128, float, PAGED, ROPE>(gh, a, span, nsubs, B, st);
      case 256: return dispatch_gh<256, float, PAGED, ROPE>(gh, a, span, nsubs, B, st);
    }
  } else {
    switch (d) {
      case 64: return dispatch_gh<64, bf16_t, PAGED, ROPE>(gh, a, span, nsubs, B, st);
      case 128: return dispatch_gh<128, bf16_t, PAGED, ROPE>(gh, a, span, nsubs, B, st);
      case 256: return dispatch_gh<256, bf16_t, PAGED, ROPE>(gh, a, span, nsubs, B, st);
    }
  }
  return MOLOT_ENOTSUP;
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

// Chunking + workspace of one launch.  `span` bounds every sequence's row
// range tiled by chunks (cache rows only when the kernel folds in the new
// token); B * nkv * subgroups workgroups share each chunk index.
int plan_launch(AttnArgs& a, int d, int span, int gh, int nsubs, int B, bool paged, int align,
                int wpc, void* stream) {
  const int rows = a.nkv * nsubs * B;
  a.chunk = plan_chunk(span > 0 ? span : 1, rows, align, wpc);
  a.nchunks = span > 0 ? (span + a.chunk - 1) / a.chunk : 1;
  // bound the chunk count (grid x, and the finishing workgroup's merge loop)
  while (a.nchunks > 4096 && a.chunk < kMaxChunk) {
    a.chunk *= 2;
    a.nchunks = (span + a.chunk - 1) / a.chunk;
  }
  if (a.nchunks > 4096) return MOLOT_ENOTSUP;
  a.part_o = nullptr;
  a.part_ml = nullptr;
  a.counters = nullptr;
  if (a.nchunks == 1 && !paged) return 0;  // single chunk: written directly
  if ((long)rows > kMaxCounters) return MOLOT_ENOTSUP;
  const size_t po = (size_t)B * a.nq * a.nchunks * d;
  const size_t pml = (size_t)B * a.nq * a.nchunks * 2;
  float* part = nullptr;
  const int st = workspace(stream, (po + pml) * sizeof(float), &a.counters, &part);
  if (st) return st;
  a.part_o = part;
  a.part_ml = part + po;
  return 0;
}

template <bool PAGED, bool ROPE>
int run_attn(AttnArgs& a, int d, int kv_dtype, int span, int B, void* stream) {
  const int G = a.nq / a.nkv;
  const int gh = pick_gh(G);
  const int nsubs = G / gh;
  return dispatch_attn<PAGED, ROPE>(d, kv_dtype, gh, a, span, nsubs, B, stream);
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

const char* molot_hip_version(void) { return "molot_amd 0.2"; }

void molot_rope_inv_freq(float base, int d, float* out) {
  for (int i = 0; i < d / 2; ++i) out[i] = 1.0f / powf(base, (2.0f * (float)i) / (float)d);
}

void molot_hip_set_split_chunk(int tokens) { g_split_chunk = tokens > 0 ? tokens : 0; }

int molot_hip_split_plan(int nkv, int n_att, int d, int kv_dtype, int* nchunks, int* chunk) {
  if (nkv <= 0 || n_att < 0 || !nchunks || !chunk || !supported_d(d)) return MOLOT_EINVAL;
  // the plan of the default GQA-4 kernels (32q/8kv-style groups)
  int align = 128, wpc = 1;
  if (d == 128 && kv_dtype == MOLOT_KV_F32) {
    using T = Tune<128, 4, float>;
    align = T::NW * T::RB;
    wpc = T::NW >= 16 ? 1 : 16 / T::NW;
  }
  const int ch = plan_chunk(n_att > 0 ? n_att : 1, nkv, align, wpc);
  *chunk = ch;
  *nchunks = n_att > 0 ? (n_att + ch - 1) / ch : 0;
  return 0;
}

void molot_hip_set_tuning(int wgs_per_cu, int variant) {
  g_wgs_per_cu = wgs_per_cu > 0 ? wgs_per_cu : 0;
  g_variant = variant > 0 ? variant : 0;
}

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
  int t0 = (window > 0 && pos_cur - window + 1 > 0) ? pos_cur - window + 1 : 0;
  if (t0 > n) t0 = n;
  const int n_att = n - t0;
  if (n_att <= 0) return zero_out(O, (int64_t)nq * d, (hipStream_t)stream);  // o = 0
  if (!K || !V) return MOLOT_EINVAL;
  const int esz = kv_dtype == MOLOT_KV_F32 ? 4 : 2;
  if (!aligned16(K) || !aligned16(V) || !aligned16(Q) || !aligned16(O) ||
      (tok_stride * esz) % 16 || (head_stride * esz) % 16)
    return MOLOT_EINVAL;  // 16-byte vector loads of every row
  AttnArgs a{};
  a.q = Q;
  a.k = const_cast<void*>(K);
  a.v = const_cast<void*>(V);
  a.o = O;
  a.tok_stride = tok_stride;
  a.head_stride = head_stride;
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
  if (!q || !k_new || !v_new || !K || !V || !O || !inv_freq || slot < 0) return MOLOT_EINVAL;
  if (!aligned16(K) || !aligned16(V) || !aligned16(q) || !aligned16(O)) return MOLOT_EINVAL;
  const int n = slot + 1;
  int t0 = (window > 0 && pos - window + 1 > 0) ? pos - window + 1 : 0;
  if (t0 > n) t0 = n;
  if (t0 > n - 1) {
    // the new token itself is outside the window: append, rotate q, o = 0
    st = molot_hip_rope_append(q, k_new, v_new, K, V, nq, nkv, d, slot, pos, inv_freq, kv_dtype,
                               stream);
    if (st) return st;
    return zero_out(O, (int64_t)nq * d, (hipStream_t)stream);
  }
  AttnArgs a{};
  a.q = q;
  a.q_out = q;
  a.k_new = k_new;
  a.v_new = v_new;
  a.k = K;
  a.v = V;
  a.inv_freq = inv_freq;
  a.o = O;
  a.tok_stride = (int64_t)nkv * d;
  a.head_stride = d;
  a.nq = nq;
  a.nkv = nkv;
  a.n = n;
  a.t0 = t0;
  a.pos = pos;
  a.window = window;
  a.scale = scale;
  return run_attn<false, true>(a, d, kv_dtype, n - 1 - t0, 1, stream);  // cache rows
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
  const int esz = kv_dtype == MOLOT_KV_F32 ? 4 : 2;
  if (((int64_t)d * esz) % 16) return MOLOT_EINVAL;
  int shift = 0;
  while ((1 << shift) < page) ++shift;
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

int molot_hip_decode_step_paged(float* q, const float* k_new, const float* v_new, void* K,
                                void* V, float* O, const int32_t* block_table,
                                const int32_t* seq_lens, const int32_t* pos, int B,
                                int max_blocks, int max_seq_len, int nq, int nkv, int d, int page,
                                const float* inv_freq, float scale, int window, int kv_dtype,
                                void* stream) {
  AttnArgs a{};
  int span = 0;
  int st = paged_args(a, q, K, V, O, block_table, seq_lens, pos, B, max_blocks, max_seq_len, nq,
                      nkv, d, page, scale, window, kv_dtype, &span);
  if (st) return st;
  if (!k_new || !v_new || !inv_freq) return MOLOT_EINVAL;
  if (B == 0) return 0;
  if (pos) {
    // a position behind the cache end can leave the new slot outside the
    // window; the split path only folds in rows it attends, so take the
    // unfused kernels there (append, then attention over the cache)
    st = molot_hip_rope_append_paged(q, k_new, v_new, K, V, block_table, seq_lens, pos, B,
                                     max_blocks, nq, nkv, d, page, inv_freq, kv_dtype, stream);
    if (st) return st;
    return run_attn<true, false>(a, d, kv_dtype, span, B, stream);
  }
  a.q_out = q;
  a.k_new = k_new;
  a.v_new = v_new;
  a.inv_freq = inv_freq;
  return run_attn<true, true>(a, d, kv_dtype, span, B, stream);  // span >= cache rows
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
