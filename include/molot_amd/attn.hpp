// Header-only C++ layer over the molot_amd C ABI (include/molot_amd/attn_hip.h).
//
// Drop-ins with the reference's own signatures, for a Molot-style host
// forward pass whose KV cache lives in device memory:
//   molot::amd::attn_decode_gqa_cache  <- include/molot/attn.h:125-127
//   molot::amd::attn_decode_gqa        <- include/molot/attn.h:111-113
//   molot::amd::rope_apply             <- include/molot/attn.h:19
//   molot::amd::rope_inv_freq          <- include/molot/attn.h:31
//   molot::amd::DeviceKV               <- Runner::KVC, include/molot/forward.h:48-51,
//                                         with the decode block forward.h:554-591
//                                         and the prefill block :367-399, for
//                                         layers with their own KV and layers
//                                         reading another layer's (shared KV)
// The reference's ThreadPool& argument is accepted and ignored.  Calls are
// synchronous like the reference's (outputs are valid on return); Q/O may be
// host or device pointers (host ones are staged through per-thread device
// buffers), K/V must be device pointers.  Errors throw std::runtime_error, as
// the reference's caller does (forward.h:570, :580).
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstddef>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "molot_amd/attn_hip.h"

namespace molot {
class ThreadPool;  // the reference's pool type (include/molot/thread_pool.h)
}

namespace molot::amd {

inline void check(int status, const char* what) {
  if (status != 0) throw std::runtime_error(std::string(what) + ": " + molot_hip_strerror(status));
}

inline void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// True for device (or managed) memory, false for host memory.
inline bool is_device_ptr(const void* p) {
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
    (void)hipGetLastError();  // unregistered host memory reports an error
    return false;
  }
  return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged;
}

// Per-thread staging for host-side vectors (small: q, the new k and v rows,
// o): a device buffer and a pinned host mirror of the same size, grown when
// a call needs more (calls are synchronous, so nothing is in flight then).
class Staging {
 public:
  ~Staging() {
    if (dev_) (void)hipFree(dev_);
    if (host_) (void)hipHostFree(host_);
  }
  void reserve(size_t floats) {
    if (floats <= cap_) return;
    if (dev_) check_hip(hipFree(dev_), "hipFree");
    if (host_) check_hip(hipHostFree(host_), "hipHostFree");
    dev_ = host_ = nullptr;
    cap_ = 0;
    check_hip(hipMalloc(&dev_, floats * sizeof(float)), "hipMalloc");
    check_hip(hipHostMalloc(&host_, floats * sizeof(float), hipHostMallocDefault),
              "hipHostMalloc");
    cap_ = floats;
  }
  float* dev() { return static_cast<float*>(dev_); }
  float* host() { return static_cast<float*>(host_); }
  static Staging& local() {
    static thread_local Staging s;
    return s;
  }

 private:
  void* dev_ = nullptr;
  void* host_ = nullptr;
  size_t cap_ = 0;
};

// Device views of one call's vectors: the caller's pointers where they are
// device memory; host ones packed into the thread's pinned mirror as
// [k | v | q | o] (the host ones only, each slot on 16 bytes), so that the
// inputs go over in one copy and q (rotated, for a decode step) and o come
// back in one.  `finish` copies back, waits and unpacks.
struct CallStage {
  float* q;  // device views
  float* o;
  const float* k = nullptr;
  const float* v = nullptr;

  CallStage(float* Q, bool q_rotated, float* O, size_t qn, size_t on, hipStream_t s,
            const float* K = nullptr, const float* V = nullptr, size_t kn = 0)
      : q(Q), o(O), k(K), v(V), s_(s), q_user_(Q), o_user_(O), qn_(qn), on_(on) {
    const bool kh = K && !is_device_ptr(K), vh = V && !is_device_ptr(V);
    qh_ = !is_device_ptr(Q);
    oh_ = !is_device_ptr(O);
    q_back_ = qh_ && q_rotated;
    // every slot starts on 16 bytes (the C ABI's alignment of its vectors)
    auto up4 = [](size_t n) { return (n + 3) & ~size_t(3); };
    const size_t in = (kh ? up4(kn) : 0) + (vh ? up4(kn) : 0) + (qh_ ? up4(qn) : 0);
    const size_t total = in + (oh_ ? up4(on) : 0);
    if (total == 0) return;
    staged_ = true;
    Staging& st = Staging::local();
    st.reserve(total);
    float* hb = st.host();
    float* db = st.dev();
    size_t off = 0;
    auto pack = [&](const float* src, size_t n) {
      std::memcpy(hb + off, src, n * sizeof(float));
      off += up4(n);
      return db + off - up4(n);
    };
    if (kh) k = pack(K, kn);
    if (vh) v = pack(V, kn);
    if (qh_) {
      q_off_ = off;
      q = pack(Q, qn);
    }
    if (in) check_hip(hipMemcpyAsync(db, hb, in * sizeof(float), hipMemcpyHostToDevice, s), "H2D");
    if (oh_) {
      o_off_ = off;
      o = db + off;
    }
    // what comes back: q (when rotated) and o, adjacent in the mirror
    back_beg_ = q_back_ ? q_off_ : o_off_;
    back_end_ = oh_ ? o_off_ + on : (q_back_ ? q_off_ + qn : back_beg_);
  }
  // a call that threw before finish: nothing may still read the mirror when
  // the next call packs it
  ~CallStage() {
    if (staged_ && !finished_) (void)hipStreamSynchronize(s_);
  }
  void finish() {
    finished_ = true;
    Staging& st = Staging::local();
    if ((oh_ || q_back_) && back_end_ > back_beg_)
      check_hip(hipMemcpyAsync(st.host() + back_beg_, st.dev() + back_beg_,
                               (back_end_ - back_beg_) * sizeof(float), hipMemcpyDeviceToHost, s_),
                "D2H");
    check_hip(hipStreamSynchronize(s_), "hipStreamSynchronize");
    if (q_back_) std::memcpy(q_user_, st.host() + q_off_, qn_ * sizeof(float));
    if (oh_) std::memcpy(o_user_, st.host() + o_off_, on_ * sizeof(float));
  }

 private:
  hipStream_t s_;
  float* q_user_;
  float* o_user_;
  size_t qn_, on_;
  bool qh_ = false, oh_ = false, q_back_ = false, staged_ = false, finished_ = false;
  size_t q_off_ = 0, o_off_ = 0, back_beg_ = 0, back_end_ = 0;
};

// attn.h:31-33
inline void rope_inv_freq(float base, int d, float* out) { molot_rope_inv_freq(base, d, out); }

// attn.h:19-28 on one device-resident head x[d]; inv_freq is a device table.
inline void rope_apply(float* x, int d, int pos, const float* inv_freq, hipStream_t s = nullptr) {
  check(molot_hip_rope_apply(x, 1, d, pos, inv_freq, s), "rope_apply");
  check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
}

// attn.h:125-127: K, V device pointers to the [n][nkv*qhd] fp32 cache.
inline void attn_decode_gqa_cache(const float* Q, const float* K, const float* V, float* O, int nq,
                                  int nkv, int n, int qhd, float scale, int pos_cur, int window,
                                  ThreadPool& /*pool*/, hipStream_t s = nullptr) {
  CallStage v(const_cast<float*>(Q), false, O, (size_t)nq * qhd, (size_t)nq * qhd, s);
  check(molot_hip_attn_decode_gqa_cache(v.q, K, V, v.o, nq, nkv, n, qhd, scale, pos_cur, window,
                                        MOLOT_KV_F32, s),
        "attn_decode_gqa_cache");
  v.finish();
}

// attn.h:111-113: head-major [nkv][n][d] device K, V.
inline void attn_decode_gqa(const float* Q, const float* K, const float* V, float* O, int nq,
                            int nkv, int n, int d, float scale, ThreadPool& /*pool*/,
                            hipStream_t s = nullptr) {
  CallStage v(const_cast<float*>(Q), false, O, (size_t)nq * d, (size_t)nq * d, s);
  check(molot_hip_attn_decode_gqa(v.q, K, V, v.o, nq, nkv, n, d, scale, MOLOT_KV_F32, s),
        "attn_decode_gqa");
  v.finish();
}

// The layer's norms of the fresh q, k, v (forward.h:554, 562-563): the
// weights are device tables of hd floats (L.q_norm, L.k_norm); NULL skips
// that norm; v_norm is hp.v_norm and eps hp.eps.
struct LayerNorms {
  const float* q_norm = nullptr;
  const float* k_norm = nullptr;
  bool v_norm = false;
  float eps = 1e-6f;
};

// Device KV cache of one layer (Runner::KVC, forward.h:48-51) with the
// decode-attention block of forward.h:554-591 in one fused launch, the
// layer prefill (forward.h:367-399), and the same blocks for layers that
// read this cache as shared KV (forward.h:578-591, :394-398).
class DeviceKV {
 public:
  int n = 0, cap = 0, nkv = 0, hd = 0, kv_dtype = MOLOT_KV_F32;
  void* k = nullptr;  // [cap][nkv*hd]
  void* v = nullptr;

  DeviceKV(int cap_, int nkv_, int hd_, int kv_dtype_ = MOLOT_KV_F32)
      : cap(cap_), nkv(nkv_), hd(hd_), kv_dtype(kv_dtype_) {
    const size_t bytes =
        kv_dtype == MOLOT_KV_Q8
            ? (size_t)cap * (size_t)molot_hip_q8_row_bytes(nkv, hd)
            : (size_t)cap * nkv * hd * (kv_dtype == MOLOT_KV_F32 ? 4 : 2);
    check_hip(hipMalloc(&k, bytes), "hipMalloc K");
    check_hip(hipMalloc(&v, bytes), "hipMalloc V");
    check_hip(hipMemset(k, 0, bytes), "hipMemset K");
    check_hip(hipMemset(v, 0, bytes), "hipMemset V");
  }
  ~DeviceKV() {
    if (k) (void)hipFree(k);
    if (v) (void)hipFree(v);
  }
  DeviceKV(const DeviceKV&) = delete;
  DeviceKV& operator=(const DeviceKV&) = delete;

  void reset() { n = 0; }  // molot_chat.cc /reset

  // forward.h:556-591 for a layer that owns its KV: q (nq heads) rotated in
  // place, k rotated and appended with v at slot n, n++, then attention into
  // ao.  q, k, v, ao may be host or device pointers; inv_freq is a device
  // table of hd/2 floats (the layer's L.freq), or NULL for a layer without
  // RoPE (an empty L.freq: forward.h:556, :566 skip the rotation).
  void decode(float* q, const float* knew, const float* vnew, float* ao, int nq, int pos,
              const float* inv_freq, float scale, int window, hipStream_t s = nullptr) {
    decode(q, knew, vnew, ao, nq, pos, inv_freq, scale, window, LayerNorms{}, s);
  }

  // forward.h:554-591: the same with the layer's norms of q, k and v fused
  // into the launch (before RoPE and the append, as forward.h orders them).
  void decode(float* q, const float* knew, const float* vnew, float* ao, int nq, int pos,
              const float* inv_freq, float scale, int window, const LayerNorms& nm,
              hipStream_t s = nullptr) {
    if (n >= cap) throw std::runtime_error("fwd: KV cache full");  // forward.h:570
    const size_t qf = (size_t)nq * hd, kf = (size_t)nkv * hd;
    CallStage view(q, true, ao, qf, qf, s, knew, vnew, kf);
    if (nm.q_norm || nm.k_norm || nm.v_norm)
      check(molot_hip_decode_step_norm(view.q, view.k, view.v, k, v, view.o, nq, nkv, hd, n, pos,
                                       nm.q_norm, nm.k_norm, nm.v_norm ? 1 : 0, nm.eps, inv_freq,
                                       scale, window, kv_dtype, s),
            "decode_step_norm");
    else
      check(molot_hip_decode_step(view.q, view.k, view.v, k, v, view.o, nq, nkv, hd, n, pos,
                                  inv_freq, scale, window, kv_dtype, s),
            "decode_step");
    ++n;
    view.finish();
  }

  // forward.h:554-558 and 578-591 for a layer without its own KV (L.has_kv
  // false) reading this cache: q (nq heads) normed with nm.q_norm and
  // rotated at pos (inv_freq NULL: a layer without RoPE) in place, then
  // attention over this cache's n slots into ao; nothing appended.  q, ao
  // may be host or device pointers.
  void decode_shared(float* q, float* ao, int nq, int pos, const float* inv_freq, float scale,
                     int window, const LayerNorms& nm = LayerNorms{},
                     hipStream_t s = nullptr) const {
    if (n == 0) throw std::runtime_error("fwd: shared KV empty");  // forward.h:580
    CallStage view(q, true, ao, (size_t)nq * hd, (size_t)nq * hd, s);
    check(molot_hip_decode_step_shared(view.q, k, v, view.o, nq, nkv, hd, n, pos, nm.q_norm,
                                       nm.eps, inv_freq, scale, window, kv_dtype, s),
          "decode_step_shared");
    view.finish();
  }

  // forward.h:367-399 for a layer that owns this cache: M prompt tokens'
  // Q [M][nq][hd] (normed, rotated in place), K_new/V_new [M][nkv][hd]
  // (normed, rotated, appended at slots n .. n+M-1), AO [M][nq][hd]: device
  // pointers.  Positions pos0 .. pos0+M-1; asynchronous on s.
  void prefill(float* Q, const float* K_new, const float* V_new, float* AO, int nq, int M,
               int pos0, const float* inv_freq, float scale, int window,
               const LayerNorms& nm = LayerNorms{}, hipStream_t s = nullptr) {
    if (n + M > cap) throw std::runtime_error("fwd: KV cache full");  // forward.h:385
    check(molot_hip_prefill_step(Q, K_new, V_new, k, v, AO, nq, nkv, hd, M, n, pos0, nm.q_norm,
                                 nm.k_norm, nm.v_norm ? 1 : 0, nm.eps, inv_freq, scale, window,
                                 kv_dtype, s),
          "prefill_step");
    n += M;
  }

  // forward.h:367-399 for a layer without its own KV reading this cache
  // (which already holds the prompt: the source layer ran first): Q
  // [M][nq][hd] normed and rotated in place, causal attention over this
  // cache's n slots into AO; device pointers, asynchronous on s.
  void prefill_shared(float* Q, float* AO, int nq, int M, int pos0, const float* inv_freq,
                      float scale, int window, const LayerNorms& nm = LayerNorms{},
                      hipStream_t s = nullptr) const {
    check(molot_hip_prefill_q(Q, nq, hd, M, pos0, nm.q_norm, nm.eps, inv_freq, s), "prefill_q");
    check(molot_hip_attn_prefill_gqa(Q, k, v, AO, nq, nkv, M, n, hd, scale, pos0, window,
                                     kv_dtype, s),
          "attn_prefill_gqa");
  }

  // forward.h:589-590 alone (attention over this cache, q as given).
  void attend(const float* q, float* ao, int nq, float scale, int pos_cur, int window,
              hipStream_t s = nullptr) const {
    if (n == 0) throw std::runtime_error("fwd: shared KV empty");  // forward.h:580
    CallStage view(const_cast<float*>(q), false, ao, (size_t)nq * hd, (size_t)nq * hd, s);
    check(molot_hip_attn_decode_gqa_cache(view.q, k, v, view.o, nq, nkv, n, hd, scale, pos_cur,
                                          window, kv_dtype, s),
          "attn_decode_gqa_cache");
    view.finish();
  }

};

}  // namespace molot::amd
