// Self-check of the paged-KV manager (include/molot_amd/paged_kv.hpp) on
// the GPU: sequences prefilled and decoded as a continuous batch across two
// layers, one freed and its blocks reused by a new one, against the CPU
// oracle (oracle/attn_oracle.c) on per-sequence contiguous caches.  The
// oracle's attention runs on the rows the GPU appended (read back from the
// pages) after those rows are checked against the oracle's own append, so
// the output comparison isolates the attention.  Run by
// tests/test_cpp_layer.py.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <vector>

#include "attn_oracle.h"
#include "check_util.hpp"
#include "molot_amd/paged_kv.hpp"

namespace {

constexpr int kLayers = 2, kNq = 8, kNkv = 2, kD = 128, kPage = 16, kBlocks = 40, kCap = 512;
constexpr float kEps = 1e-6f, kScale = 0.088f;

float bf2f(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// one sequence's oracle state: a contiguous bf16 cache per layer
struct RefSeq {
  int len = 0;
  std::vector<std::vector<uint16_t>> K, V;
  RefSeq() : K(kLayers, std::vector<uint16_t>((size_t)kCap * kNkv * kD)),
             V(kLayers, std::vector<uint16_t>((size_t)kCap * kNkv * kD)) {}
};

struct Dev {
  float* p = nullptr;
  size_t n = 0;
  explicit Dev(size_t floats) : n(floats) {
    molot::amd::check_hip(hipMalloc(&p, floats * 4), "hipMalloc");
  }
  ~Dev() { (void)hipFree(p); }
  void put(const std::vector<float>& h) {
    molot::amd::check_hip(hipMemcpy(p, h.data(), h.size() * 4, hipMemcpyHostToDevice), "H2D");
  }
  std::vector<float> get(size_t floats) const {
    std::vector<float> h(floats);
    molot::amd::check_hip(hipMemcpy(h.data(), p, floats * 4, hipMemcpyDeviceToHost), "D2H");
    return h;
  }
};

// norms (when given) and rope of one token's q [nq][d] and k [nkv][d], v
// normed over all its values: forward.h:554-568 from the oracle's parts
void ref_token(float* q, float* k, float* v, int pos, const float* inv, const float* qn,
               const float* kn, bool vn) {
  for (int h = 0; h < kNq; ++h)
    if (qn) orc_rmsnorm(q + h * kD, qn, q + h * kD, kD, kEps);
  orc_rope_apply_heads(q, kNq, kD, pos, inv);
  for (int h = 0; h < kNkv; ++h)
    if (kn) orc_rmsnorm(k + h * kD, kn, k + h * kD, kD, kEps);
  if (vn) orc_rmsnorm(v, nullptr, v, kNkv * kD, kEps);
  orc_rope_apply_heads(k, kNkv, kD, pos, inv);
}

// Reads rows [r0, r1) of sequence `blocks` from a layer's bf16 pages.
std::vector<uint16_t> read_rows(const molot::amd::PagedKVCache& kv, void* pages,
                                const std::vector<int>& blocks, int r0, int r1) {
  std::vector<uint16_t> out((size_t)(r1 - r0) * kNkv * kD);
  for (int t = r0; t < r1; ++t)
    for (int h = 0; h < kNkv; ++h) {
      const size_t off = (((size_t)blocks[t / kPage] * kNkv + h) * kPage + t % kPage) * kD;
      molot::amd::check_hip(hipMemcpy(out.data() + ((size_t)(t - r0) * kNkv + h) * kD,
                                      (const uint16_t*)pages + off, kD * 2,
                                      hipMemcpyDeviceToHost),
                            "D2H row");
    }
  return out;
}

// The GPU's appended rows match the oracle's own append to a bf16 ulp (the
// normed, rotated fp32 values may differ by an fp32 ulp before rounding),
// then replace them so the attention is compared on identical caches.
double adopt_rows(RefSeq& r, int layer, const std::vector<uint16_t>& gk,
                  const std::vector<uint16_t>& gv, int r0, int r1) {
  double worst = 0;
  for (int side = 0; side < 2; ++side) {
    std::vector<uint16_t>& C = side ? r.V[layer] : r.K[layer];
    const std::vector<uint16_t>& G = side ? gv : gk;
    for (size_t i = 0; i < G.size(); ++i) {
      const float a = bf2f(C[(size_t)r0 * kNkv * kD + i]), b = bf2f(G[i]);
      worst = std::fmax(worst, std::fabs(a - b) / std::fmax(1.0f, std::fabs(a)));
      C[(size_t)r0 * kNkv * kD + i] = G[i];
    }
  }
  (void)r1;
  return worst;
}

}  // namespace

int main() {
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) {
    std::printf("no GPU\n");
    return 2;
  }
  Rng rng(2024);
  std::vector<float> inv(kD / 2), qn(kD), kn(kD);
  orc_rope_inv_freq(500000.0f, kD, inv.data());
  rng.normal(qn);
  rng.normal(kn);
  for (int i = 0; i < kD; ++i) {
    qn[i] = 1.0f + 0.2f * qn[i];
    kn[i] = 1.0f + 0.2f * kn[i];
  }
  Dev d_inv(kD / 2), d_w(2 * kD);
  d_inv.put(inv);
  std::vector<float> w2(qn);
  w2.insert(w2.end(), kn.begin(), kn.end());
  d_w.put(w2);
  // layer 0 with the layer norms, layer 1 without (both paths)
  molot::amd::LayerNorms norms[kLayers];
  norms[0].q_norm = d_w.p;
  norms[0].k_norm = d_w.p + kD;
  norms[0].v_norm = true;
  norms[0].eps = kEps;

  molot::amd::PagedKVCache kv(kLayers, kBlocks, kNkv, kD, kPage, MOLOT_KV_BF16);
  std::vector<RefSeq> ref(8);
  double worst_o = 0, worst_row = 0;

  auto prefill = [&](int id, int M) {
    RefSeq& r = ref[id];
    const int pos0 = r.len;
    kv.begin_prefill(id, M);
    for (int l = 0; l < kLayers; ++l) {
      std::vector<float> q((size_t)M * kNq * kD), k((size_t)M * kNkv * kD),
          v((size_t)M * kNkv * kD);
      rng.normal(q);
      rng.normal(k);
      rng.normal(v);
      Dev dq(q.size()), dk(k.size()), dv(v.size()), dO(q.size());
      dq.put(q);
      dk.put(k);
      dv.put(v);
      kv.prefill(l, dq.p, dk.p, dv.p, dO.p, kNq, pos0, d_inv.p, kScale, 0, norms[l]);
      molot::amd::check_hip(hipDeviceSynchronize(), "sync");
      const bool n = norms[l].q_norm != nullptr;
      for (int m = 0; m < M; ++m) {
        float* qm = q.data() + (size_t)m * kNq * kD;
        float* km = k.data() + (size_t)m * kNkv * kD;
        float* vm = v.data() + (size_t)m * kNkv * kD;
        ref_token(qm, km, vm, pos0 + m, inv.data(), n ? qn.data() : nullptr,
                  n ? kn.data() : nullptr, n);
        orc_f32_to_bf16_array(km, r.K[l].data() + (size_t)(pos0 + m) * kNkv * kD, kNkv * kD);
        orc_f32_to_bf16_array(vm, r.V[l].data() + (size_t)(pos0 + m) * kNkv * kD, kNkv * kD);
      }
      worst_row = std::fmax(worst_row,
                            adopt_rows(r, l, read_rows(kv, kv.k_pages(l), kv.blocks(id), pos0,
                                                       pos0 + M),
                                       read_rows(kv, kv.v_pages(l), kv.blocks(id), pos0,
                                                 pos0 + M),
                                       pos0, pos0 + M));
      std::vector<float> O((size_t)M * kNq * kD);
      orc_attn_prefill(q.data(), r.K[l].data(), r.V[l].data(), O.data(), kNq, kNkv, M, pos0 + M,
                       kD, kScale, pos0, 0, ORC_KV_BF16, 0);
      worst_o = std::fmax(worst_o, normwise(dO.get(O.size()), O));
      CHECK(normwise(dq.get(q.size()), q) < 2e-6, "prefill q seq %d layer %d", id, l);
    }
    kv.end_prefill();
    r.len += M;
  };

  auto decode = [&](const std::vector<int>& ids) {
    const int B = (int)ids.size();
    kv.begin_decode(ids);
    for (int l = 0; l < kLayers; ++l) {
      std::vector<float> q((size_t)B * kNq * kD), k((size_t)B * kNkv * kD),
          v((size_t)B * kNkv * kD);
      rng.normal(q);
      rng.normal(k);
      rng.normal(v);
      Dev dq(q.size()), dk(k.size()), dv(v.size()), dO(q.size());
      dq.put(q);
      dk.put(k);
      dv.put(v);
      kv.decode(l, dq.p, dk.p, dv.p, dO.p, kNq, d_inv.p, kScale, 0, norms[l]);
      molot::amd::check_hip(hipDeviceSynchronize(), "sync");
      const std::vector<float> got = dO.get(q.size());
      const bool n = norms[l].q_norm != nullptr;
      for (int b = 0; b < B; ++b) {
        RefSeq& r = ref[ids[b]];
        float* qb = q.data() + (size_t)b * kNq * kD;
        float* kb = k.data() + (size_t)b * kNkv * kD;
        float* vb = v.data() + (size_t)b * kNkv * kD;
        ref_token(qb, kb, vb, r.len, inv.data(), n ? qn.data() : nullptr,
                  n ? kn.data() : nullptr, n);
        orc_f32_to_bf16_array(kb, r.K[l].data() + (size_t)r.len * kNkv * kD, kNkv * kD);
        orc_f32_to_bf16_array(vb, r.V[l].data() + (size_t)r.len * kNkv * kD, kNkv * kD);
        worst_row = std::fmax(worst_row,
                              adopt_rows(r, l, read_rows(kv, kv.k_pages(l), kv.blocks(ids[b]),
                                                         r.len, r.len + 1),
                                         read_rows(kv, kv.v_pages(l), kv.blocks(ids[b]), r.len,
                                                   r.len + 1),
                                         r.len, r.len + 1));
        std::vector<float> O((size_t)kNq * kD);
        orc_attn_decode(qb, r.K[l].data(), r.V[l].data(), O.data(), kNq, kNkv, r.len + 1, kD,
                        kScale, r.len, 0, ORC_KV_BF16, (int64_t)kNkv * kD, kD, 0, nullptr, 0, 0);
        std::vector<float> g(got.begin() + (size_t)b * kNq * kD,
                             got.begin() + (size_t)(b + 1) * kNq * kD);
        worst_o = std::fmax(worst_o, normwise(g, O));
      }
    }
    kv.end_decode();
    for (int id : ids) ref[id].len += 1;
  };

  const int A = kv.add_sequence(), Bq = kv.add_sequence(), C = kv.add_sequence();
  prefill(A, 20);
  prefill(Bq, 37);
  prefill(C, 5);
  for (int s = 0; s < 6; ++s) decode({A, Bq, C});
  const int freed = kv.free_blocks();
  const int b_blocks = (int)kv.blocks(Bq).size();
  kv.free_sequence(Bq);
  CHECK(kv.free_blocks() == freed + b_blocks, "freed blocks %d", kv.free_blocks());
  const int Dq = kv.add_sequence();
  CHECK(Dq == Bq, "sequence id reused (%d)", Dq);
  ref[Dq] = RefSeq{};
  prefill(Dq, 50);  // lands in B's freed blocks
  for (int s = 0; s < 4; ++s) decode({A, C, Dq});
  decode({C});
  CHECK(kv.length(A) == 30 && kv.length(C) == 16 && kv.length(Dq) == 54, "lengths %d %d %d",
        kv.length(A), kv.length(C), kv.length(Dq));
  CHECK(worst_o < 1e-5, "paged outputs vs oracle: normwise %g", worst_o);
  CHECK(worst_row <= 8e-3, "appended rows vs oracle: %g", worst_row);
  std::printf("[%s] PagedKVCache: 4 sequences, 2 layers, prefill + 11 decode steps, block "
              "reuse: max normwise err %.2e, rows within %.1e\n",
              failures ? "FAIL" : "ok", worst_o, worst_row);

  // a full pool reports what a full contiguous cache does (forward.h:570)
  {
    molot::amd::PagedKVCache small(1, 2, kNkv, kD, kPage, MOLOT_KV_BF16);
    const int s = small.add_sequence();
    bool threw = false;
    try {
      small.begin_prefill(s, 40);
    } catch (const std::runtime_error& e) {
      threw = std::strcmp(e.what(), "fwd: KV cache full") == 0;
    }
    CHECK(threw, "full pool did not throw 'fwd: KV cache full'");
  }
  std::printf(failures ? "FAILED (%d)\n" : "PASSED\n", failures);
  return failures ? 1 : 0;
}
