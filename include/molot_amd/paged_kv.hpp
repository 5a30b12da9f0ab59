// Paged KV cache with continuous batching: the host side of the paged
// kernels (include/molot_amd/attn_hip.h: molot_hip_decode_step_paged_norm,
// molot_hip_prefill_step_paged).
//
// No reference counterpart: the reference keeps one contiguous fp32 cache
// per layer and sequence (Runner::KVC, include/molot/forward.h:48-51, one
// Runner per chat); its design notes plan vLLM-style 16-token pages
// (the reference's DESIGN.md:47-48) and its README lists them as not
// implemented (the reference's README.md:112-114).  This class is that
// caller side:
//   * one pool of pages per layer, [num_blocks][nkv][page][hd] (a Q8 pool:
//     MOLOT_KV_Q8 blocks of molot_hip_q8_block_bytes each), all layers
//     sharing one block allocator, so a sequence's block ids are the same in
//     every layer;
//   * sequences are added and freed at any time (continuous batching); a
//     freed sequence's blocks return to the pool at once;
//   * a decode step runs any subset of the live sequences as one batch:
//     begin_decode uploads that batch's block table and lengths once, every
//     layer's decode() reuses them, end_decode advances the lengths;
//   * a prompt is prefilled per sequence the same way (begin_prefill,
//     prefill() per layer, end_prefill).
// Errors throw std::runtime_error; a full pool is "fwd: KV cache full", as
// forward.h:570 reports a full contiguous cache.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <stdexcept>
#include <vector>

#include "molot_amd/attn.hpp"
#include "molot_amd/attn_hip.h"

namespace molot::amd {

class PagedKVCache {
 public:
  PagedKVCache(int layers, int num_blocks, int nkv, int hd, int page = 16,
               int kv_dtype = MOLOT_KV_BF16)
      : layers_(layers), nblocks_(num_blocks), nkv_(nkv), hd_(hd), page_(page),
        kv_dtype_(kv_dtype) {
    if (layers <= 0 || num_blocks <= 0 || nkv <= 0 || hd <= 0 || page <= 0 ||
        (page & (page - 1)))
      throw std::runtime_error("PagedKVCache: bad geometry");
    const size_t esz = kv_dtype == MOLOT_KV_F32 ? 4 : 2;
    pool_bytes_ = kv_dtype == MOLOT_KV_Q8
                      ? (size_t)num_blocks * (size_t)molot_hip_q8_block_bytes(nkv, hd, page)
                      : (size_t)num_blocks * nkv * page * hd * esz;
    k_.assign(layers, nullptr);
    v_.assign(layers, nullptr);
    for (int l = 0; l < layers; ++l) {
      check_hip(hipMalloc(&k_[l], pool_bytes_), "hipMalloc K pages");
      check_hip(hipMalloc(&v_[l], pool_bytes_), "hipMalloc V pages");
    }
    for (int b = num_blocks - 1; b >= 0; --b) free_.push_back(b);
  }
  ~PagedKVCache() {
    for (void* p : k_)
      if (p) (void)hipFree(p);
    for (void* p : v_)
      if (p) (void)hipFree(p);
    if (d_table_) (void)hipFree(d_table_);
    if (h_table_) (void)hipHostFree(h_table_);
    if (uploaded_) (void)hipEventDestroy(uploaded_);
  }
  PagedKVCache(const PagedKVCache&) = delete;
  PagedKVCache& operator=(const PagedKVCache&) = delete;

  // ---- sequences ----
  int add_sequence() {
    for (size_t i = 0; i < seqs_.size(); ++i)
      if (!seqs_[i].live) {
        seqs_[i] = Seq{};
        seqs_[i].live = true;
        return (int)i;
      }
    seqs_.push_back(Seq{});
    seqs_.back().live = true;
    return (int)seqs_.size() - 1;
  }
  void free_sequence(int id) {
    Seq& s = seq(id);
    for (int b : s.blocks) free_.push_back(b);
    s = Seq{};
  }
  int length(int id) const { return seq(id).len; }
  int free_blocks() const { return (int)free_.size(); }
  const std::vector<int>& blocks(int id) const { return seq(id).blocks; }

  // ---- decode: one new token for each sequence of a batch ----
  // Reserves a slot per sequence and uploads the batch's block table
  // [B][max_blocks] and lengths (counting the new token) on stream s.
  // Throws "fwd: KV cache full" (forward.h:570) before any state of the
  // step is set when the pool cannot hold the batch's new tokens.
  void begin_decode(const std::vector<int>& ids, hipStream_t s = nullptr) {
    if (mode_ != Mode::None) throw std::runtime_error("PagedKVCache: a step is in progress");
    std::vector<int32_t> lens(ids.size());
    int maxb = 1;
    for (size_t i = 0; i < ids.size(); ++i) {
      reserve(ids[i], 1);
      lens[i] = seq(ids[i]).len + 1;
      maxb = std::max(maxb, (int)seq(ids[i]).blocks.size());
    }
    upload(ids, maxb, lens, s);
    batch_ = ids;
    mode_ = Mode::Decode;
  }
  // forward.h:554-591 for one layer over the batch: q [B][nq][hd] (normed
  // and rotated in place), k/v [B][nkv][hd] (normed, rotated, appended),
  // o [B][nq][hd]; device pointers.
  void decode(int layer, float* q, const float* k, const float* v, float* o, int nq,
              const float* inv_freq, float scale, int window, const LayerNorms& nm = LayerNorms{},
              hipStream_t s = nullptr) {
    if (mode_ != Mode::Decode) throw std::runtime_error("PagedKVCache: decode outside a step");
    check(molot_hip_decode_step_paged_norm(
              q, k, v, k_.at(layer), v_.at(layer), o, d_table_, d_lens_, nullptr,
              (int)batch_.size(), maxb_, max_len_, nq, nkv_, hd_, page_, nm.q_norm, nm.k_norm,
              nm.v_norm ? 1 : 0, nm.eps, inv_freq, scale, window, kv_dtype_, s),
          "decode_step_paged");
  }
  // forward.h:554-558, 578-591 for a layer without its own KV (L.has_kv
  // false) reading layer `src`'s pages: q normed and rotated in place
  // (inv_freq NULL: no RoPE), attention over the batch's rows, which count
  // this step's token (src appended it earlier in the step); nothing appended.
  void decode_shared(int src, float* q, float* o, int nq, const float* inv_freq, float scale,
                     int window, const LayerNorms& nm = LayerNorms{},
                     hipStream_t s = nullptr) const {
    if (mode_ != Mode::Decode) throw std::runtime_error("PagedKVCache: decode outside a step");
    check(molot_hip_decode_step_paged_shared(
              q, k_.at(src), v_.at(src), o, d_table_, d_lens_, nullptr, (int)batch_.size(), maxb_,
              max_len_, nq, nkv_, hd_, page_, nm.q_norm, nm.eps, inv_freq, scale, window,
              kv_dtype_, s),
          "decode_step_paged_shared");
  }
  // The batch's token is in every layer's pages: lengths advance by one.
  void end_decode() {
    if (mode_ != Mode::Decode) throw std::runtime_error("PagedKVCache: no decode step to end");
    for (int id : batch_) seq(id).len += 1;
    batch_.clear();
    mode_ = Mode::None;
  }

  // ---- prefill: M prompt tokens of one sequence ----
  void begin_prefill(int id, int M, hipStream_t s = nullptr) {
    if (mode_ != Mode::None) throw std::runtime_error("PagedKVCache: a step is in progress");
    if (M <= 0) throw std::runtime_error("PagedKVCache: empty prompt");
    reserve(id, M);
    batch_ = {id};
    const Seq& q = seq(id);
    upload(batch_, (int)q.blocks.size(), {q.len + M}, s);
    prefill_m_ = M;
    mode_ = Mode::Prefill;
  }
  // forward.h:367-399 for one layer: q [M][nq][hd] (normed, rotated in
  // place), k/v [M][nkv][hd], o [M][nq][hd]; positions pos0 .. pos0+M-1.
  void prefill(int layer, float* q, const float* k, const float* v, float* o, int nq, int pos0,
               const float* inv_freq, float scale, int window,
               const LayerNorms& nm = LayerNorms{}, hipStream_t s = nullptr) {
    if (mode_ != Mode::Prefill) throw std::runtime_error("PagedKVCache: prefill outside a step");
    check(molot_hip_prefill_step_paged(q, k, v, k_.at(layer), v_.at(layer), o, d_table_, maxb_,
                                       page_, nq, nkv_, hd_, prefill_m_, seq(batch_[0]).len,
                                       pos0, nm.q_norm, nm.k_norm, nm.v_norm ? 1 : 0, nm.eps,
                                       inv_freq, scale, window, kv_dtype_, s),
          "prefill_step_paged");
  }
  // forward.h:367-399 for a layer without its own KV reading layer `src`'s
  // pages: the prompt's q [M][nq][hd] normed and rotated in place, causal
  // attention over the sequence's rows so far (src appended the prompt
  // earlier in the step); nothing appended.
  void prefill_shared(int src, float* q, float* o, int nq, int pos0, const float* inv_freq,
                      float scale, int window, const LayerNorms& nm = LayerNorms{},
                      hipStream_t s = nullptr) const {
    if (mode_ != Mode::Prefill) throw std::runtime_error("PagedKVCache: prefill outside a step");
    check(molot_hip_prefill_q(q, nq, hd_, prefill_m_, pos0, nm.q_norm, nm.eps, inv_freq, s),
          "prefill_q");
    check(molot_hip_attn_prefill_paged(q, k_.at(src), v_.at(src), o, d_table_, maxb_, page_, nq,
                                       nkv_, prefill_m_, seq(batch_[0]).len + prefill_m_, hd_,
                                       scale, pos0, window, kv_dtype_, s),
          "attn_prefill_paged");
  }
  void end_prefill() {
    if (mode_ != Mode::Prefill) throw std::runtime_error("PagedKVCache: no prefill step to end");
    seq(batch_[0]).len += prefill_m_;
    batch_.clear();
    mode_ = Mode::None;
  }

  // ---- device views (tests, other kernels) ----
  void* k_pages(int layer) const { return k_.at(layer); }
  void* v_pages(int layer) const { return v_.at(layer); }
  int layers() const { return layers_; }
  int num_blocks() const { return nblocks_; }
  int page() const { return page_; }
  int kv_dtype() const { return kv_dtype_; }

 private:
  struct Seq {
    bool live = false;
    int len = 0;
    std::vector<int> blocks;
  };
  enum class Mode { None, Decode, Prefill };

  Seq& seq(int id) {
    if (id < 0 || id >= (int)seqs_.size() || !seqs_[id].live)
      throw std::runtime_error("PagedKVCache: no such sequence");
    return seqs_[id];
  }
  const Seq& seq(int id) const {
    if (id < 0 || id >= (int)seqs_.size() || !seqs_[id].live)
      throw std::runtime_error("PagedKVCache: no such sequence");
    return seqs_[id];
  }
  // Blocks for `tokens` more tokens of sequence id, from the shared pool.
  void reserve(int id, int tokens) {
    Seq& s = seq(id);
    const int need = (s.len + tokens + page_ - 1) / page_;
    if (need - (int)s.blocks.size() > (int)free_.size())
      throw std::runtime_error("fwd: KV cache full");
    while ((int)s.blocks.size() < need) {
      s.blocks.push_back(free_.back());
      free_.pop_back();
    }
  }
  // The batch's block table [B][maxb] and lengths to the device, through a
  // pinned staging buffer whose previous copy has finished (event).
  void upload(const std::vector<int>& ids, int maxb, const std::vector<int32_t>& lens,
              hipStream_t s) {
    const size_t B = ids.size();
    const size_t n = B * maxb + B, bytes = n * sizeof(int32_t);
    if (uploaded_) check_hip(hipEventSynchronize(uploaded_), "hipEventSynchronize");
    if (bytes > table_cap_) {
      // the previous step's kernels may still read the old table
      if (d_table_) check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
      if (d_table_) check_hip(hipFree(d_table_), "hipFree");
      if (h_table_) check_hip(hipHostFree(h_table_), "hipHostFree");
      d_table_ = nullptr;
      h_table_ = nullptr;
      check_hip(hipMalloc(&d_table_, bytes), "hipMalloc block table");
      check_hip(hipHostMalloc((void**)&h_table_, bytes, hipHostMallocDefault), "hipHostMalloc");
      table_cap_ = bytes;
    }
    std::fill(h_table_, h_table_ + n, 0);
    max_len_ = 0;
    for (size_t i = 0; i < B; ++i) {
      const Seq& q = seq(ids[i]);
      for (size_t j = 0; j < q.blocks.size(); ++j) h_table_[i * maxb + j] = q.blocks[j];
      h_table_[B * maxb + i] = lens[i];
      max_len_ = std::max(max_len_, (int)lens[i]);
    }
    check_hip(hipMemcpyAsync(d_table_, h_table_, bytes, hipMemcpyHostToDevice, s),
              "H2D block table");
    if (!uploaded_) check_hip(hipEventCreate(&uploaded_), "hipEventCreate");
    check_hip(hipEventRecord(uploaded_, s), "hipEventRecord");
    d_lens_ = d_table_ + B * maxb;
    maxb_ = maxb;
  }

  int layers_, nblocks_, nkv_, hd_, page_, kv_dtype_;
  size_t pool_bytes_ = 0;
  std::vector<void*> k_, v_;
  std::vector<int> free_;
  std::vector<Seq> seqs_;
  std::vector<int> batch_;
  Mode mode_ = Mode::None;
  int prefill_m_ = 0;
  int32_t* d_table_ = nullptr;
  int32_t* h_table_ = nullptr;
  hipEvent_t uploaded_ = nullptr;
  int32_t* d_lens_ = nullptr;
  size_t table_cap_ = 0;
  int maxb_ = 1, max_len_ = 0;
};

}  // namespace molot::amd
