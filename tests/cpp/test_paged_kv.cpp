// Self-check of the paged-KV manager (include/molot_amd/paged_kv.hpp) on
// the GPU: sequences prefilled and decoded as a continuous batch across two
// layers and a third layer reading layer 0's pages (shared KV), one freed
// and its blocks reused by a new one, the step state machine, against the CPU
// oracle (oracle/attn_oracle.c) on per-sequence contiguous caches of the
// same element type -- once over bf16 pages and once over Q8 pages.  The
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

// The byte formats of one token's KV row: bf16 [nkv][d], or a token-major
// Q8 row ([nkv][d] codes, then the nkv fp32 scales, padded to 16 bytes).
struct Fmt {
  int kv_dtype;
  size_t row_bytes() const {
    return kv_dtype == MOLOT_KV_Q8 ? (size_t)orc_q8_row_bytes(kNkv, kD) : (size_t)kNkv * kD * 2;
  }
  // oracle append of fp32 rows x [nkv][d] into token t of cache C
  void store(std::vector<uint8_t>& C, int t, const float* x) const {
    if (kv_dtype == MOLOT_KV_Q8)
      orc_q8_store_token(C.data(), t, x, kNkv, kD);
    else
      orc_f32_to_bf16_array(x, (uint16_t*)(C.data() + (size_t)t * row_bytes()), kNkv * kD);
  }
  // fp32 value of element (h, i) of a row
  float value(const uint8_t* row, int h, int i) const {
    if (kv_dtype == MOLOT_KV_Q8) {
      float s;
      std::memcpy(&s, row + (size_t)kNkv * kD + 4 * h, 4);
      return (float)(int8_t)row[(size_t)h * kD + i] * s;
    }
    uint16_t b;
    std::memcpy(&b, row + ((size_t)h * kD + i) * 2, 2);
    return bf2f(b);
  }
  // the step between neighbouring values of head h's row (bf16: relative)
  float step(const uint8_t* row, int h) const {
    if (kv_dtype == MOLOT_KV_Q8) {
      float s;
      std::memcpy(&s, row + (size_t)kNkv * kD + 4 * h, 4);
      return s;
    }
    return 0.f;
  }
  // token t of a sequence from its pages (blocks) into a token-major row
  void read_row(const void* pages, const std::vector<int>& blocks, int t, uint8_t* out) const {
    const size_t blk = (size_t)blocks[t / kPage];
    const int sl = t % kPage;
    for (int h = 0; h < kNkv; ++h) {
      if (kv_dtype == MOLOT_KV_Q8) {
        const size_t bb = (size_t)molot_hip_q8_block_bytes(kNkv, kD, kPage);
        const char* base = (const char*)pages + blk * bb;
        molot::amd::check_hip(hipMemcpy(out + (size_t)h * kD,
                                        base + ((size_t)h * kPage + sl) * kD, kD,
                                        hipMemcpyDeviceToHost),
                              "D2H codes");
        molot::amd::check_hip(
            hipMemcpy(out + (size_t)kNkv * kD + 4 * h,
                      base + (size_t)kNkv * kPage * kD + 4 * ((size_t)h * kPage + sl), 4,
                      hipMemcpyDeviceToHost),
            "D2H scale");
      } else {
        const size_t off = ((blk * kNkv + h) * kPage + sl) * kD * 2;
        molot::amd::check_hip(hipMemcpy(out + (size_t)h * kD * 2, (const char*)pages + off,
                                        kD * 2, hipMemcpyDeviceToHost),
                              "D2H row");
      }
    }
  }
};

// one sequence's oracle state: a contiguous cache per layer
struct RefSeq {
  int len = 0;
  std::vector<std::vector<uint8_t>> K, V;
  explicit RefSeq(const Fmt& f = Fmt{MOLOT_KV_BF16})
      : K(kLayers, std::vector<uint8_t>((size_t)kCap * f.row_bytes())),
        V(kLayers, std::vector<uint8_t>((size_t)kCap * f.row_bytes())) {}
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

// The GPU's appended rows [r0, r1) of one layer against the oracle's own
// append, then copied over it so the attention is compared on identical
// caches.  The normed, rotated fp32 values may differ by an fp32 ulp before
// rounding: bf16 rows agree to a bf16 ulp (relative), Q8 rows to one code
// (a scale may differ by an ulp, and a value on a rounding midpoint round
// the other way).  Returns the worst deviation in those units.
double adopt_rows(const Fmt& f, RefSeq& r, int layer, const molot::amd::PagedKVCache& kv,
                  const std::vector<int>& blocks, int r0, int r1) {
  const size_t R = f.row_bytes();
  std::vector<uint8_t> g(R);
  double worst = 0;
  for (int side = 0; side < 2; ++side) {
    std::vector<uint8_t>& C = side ? r.V[layer] : r.K[layer];
    const void* pages = side ? kv.v_pages(layer) : kv.k_pages(layer);
    for (int t = r0; t < r1; ++t) {
      f.read_row(pages, blocks, t, g.data());
      uint8_t* c = C.data() + (size_t)t * R;
      for (int h = 0; h < kNkv; ++h) {
        const float unit = f.kv_dtype == MOLOT_KV_Q8 ? std::fmax(f.step(c, h), f.step(g.data(), h))
                                                     : 0.f;
        for (int i = 0; i < kD; ++i) {
          const float a = f.value(c, h, i), b = f.value(g.data(), h, i);
          const double d = f.kv_dtype == MOLOT_KV_Q8
                               ? std::fabs(a - b) / (1.0001 * unit)
                               : std::fabs(a - b) / std::fmax(1.0f, std::fabs(a)) / 8e-3;
          worst = std::fmax(worst, d);
        }
      }
      std::memcpy(c, g.data(), R);
    }
  }
  return worst;
}

int run_scenario(int kv_dtype, const char* name) {
  const int failures0 = failures;
  const Fmt f{kv_dtype};
  const int odt = kv_dtype == MOLOT_KV_Q8 ? ORC_KV_Q8 : ORC_KV_BF16;
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

  molot::amd::PagedKVCache kv(kLayers, kBlocks, kNkv, kD, kPage, kv_dtype);
  std::vector<RefSeq> ref(8, RefSeq(f));
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
        f.store(r.K[l], pos0 + m, km);
        f.store(r.V[l], pos0 + m, vm);
      }
      worst_row = std::fmax(worst_row, adopt_rows(f, r, l, kv, kv.blocks(id), pos0, pos0 + M));
      std::vector<float> O((size_t)M * kNq * kD);
      orc_attn_prefill(q.data(), r.K[l].data(), r.V[l].data(), O.data(), kNq, kNkv, M, pos0 + M,
                       kD, kScale, pos0, 0, odt, 0);
      worst_o = std::fmax(worst_o, normwise(dO.get(O.size()), O));
      CHECK(normwise(dq.get(q.size()), q) < 2e-6, "%s prefill q seq %d layer %d", name, id, l);
    }
    {  // a layer reading layer 0's pages (shared KV): q norm + RoPE, no append
      std::vector<float> q((size_t)M * kNq * kD);
      rng.normal(q);
      Dev dq(q.size()), dO(q.size());
      dq.put(q);
      molot::amd::LayerNorms sn;
      sn.q_norm = d_w.p;
      sn.eps = kEps;
      kv.prefill_shared(0, dq.p, dO.p, kNq, pos0, d_inv.p, kScale, 0, sn);
      molot::amd::check_hip(hipDeviceSynchronize(), "sync");
      orc_prefill_q(q.data(), kNq, kD, M, pos0, qn.data(), kEps, inv.data());
      std::vector<float> O((size_t)M * kNq * kD);
      orc_attn_prefill(q.data(), r.K[0].data(), r.V[0].data(), O.data(), kNq, kNkv, M, pos0 + M,
                       kD, kScale, pos0, 0, odt, 0);
      worst_o = std::fmax(worst_o, normwise(dO.get(O.size()), O));
      CHECK(normwise(dq.get(q.size()), q) < 2e-6, "%s shared prefill q seq %d", name, id);
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
        f.store(r.K[l], r.len, kb);
        f.store(r.V[l], r.len, vb);
        worst_row =
            std::fmax(worst_row, adopt_rows(f, r, l, kv, kv.blocks(ids[b]), r.len, r.len + 1));
        std::vector<float> O((size_t)kNq * kD);
        orc_attn_decode(qb, r.K[l].data(), r.V[l].data(), O.data(), kNq, kNkv, r.len + 1, kD,
                        kScale, r.len, 0, odt, (int64_t)kNkv * kD, kD, 0, nullptr, 0, 0);
        std::vector<float> g(got.begin() + (size_t)b * kNq * kD,
                             got.begin() + (size_t)(b + 1) * kNq * kD);
        worst_o = std::fmax(worst_o, normwise(g, O));
      }
    }
    {  // a layer reading layer 0's pages (shared KV): its rows count this token
      std::vector<float> q((size_t)B * kNq * kD);
      rng.normal(q);
      Dev dq(q.size()), dO(q.size());
      dq.put(q);
      molot::amd::LayerNorms sn;
      sn.q_norm = d_w.p;
      sn.eps = kEps;
      kv.decode_shared(0, dq.p, dO.p, kNq, d_inv.p, kScale, 0, sn);
      molot::amd::check_hip(hipDeviceSynchronize(), "sync");
      const std::vector<float> got = dO.get(q.size()), gq = dq.get(q.size());
      for (int b = 0; b < B; ++b) {
        RefSeq& r = ref[ids[b]];
        float* qb = q.data() + (size_t)b * kNq * kD;
        std::vector<float> O((size_t)kNq * kD);
        orc_decode_step_shared(qb, r.K[0].data(), r.V[0].data(), O.data(), kNq, kNkv, kD,
                               r.len + 1, r.len, qn.data(), kEps, inv.data(), kScale, 0, odt, 0);
        std::vector<float> g(got.begin() + (size_t)b * kNq * kD,
                             got.begin() + (size_t)(b + 1) * kNq * kD);
        worst_o = std::fmax(worst_o, normwise(g, O));
        std::vector<float> gqb(gq.begin() + (size_t)b * kNq * kD,
                               gq.begin() + (size_t)(b + 1) * kNq * kD);
        std::vector<float> rq(qb, qb + (size_t)kNq * kD);
        CHECK(normwise(gqb, rq) < 2e-6, "%s shared decode q seq %d", name, ids[b]);
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
  CHECK(kv.free_blocks() == freed + b_blocks, "%s freed blocks %d", name, kv.free_blocks());
  const int Dq = kv.add_sequence();
  CHECK(Dq == Bq, "%s sequence id reused (%d)", name, Dq);
  ref[Dq] = RefSeq(f);
  prefill(Dq, 50);  // lands in B's freed blocks
  for (int s = 0; s < 4; ++s) decode({A, C, Dq});
  decode({C});
  CHECK(kv.length(A) == 30 && kv.length(C) == 16 && kv.length(Dq) == 54, "%s lengths %d %d %d",
        name, kv.length(A), kv.length(C), kv.length(Dq));
  CHECK(worst_o < 1e-5, "%s paged outputs vs oracle: normwise %g", name, worst_o);
  CHECK(worst_row <= 1.0, "%s appended rows vs oracle: %g of the allowed deviation", name,
        worst_row);
  std::printf("[%s] PagedKVCache %s: 4 sequences, 2 layers, prefill + 11 decode steps, block "
              "reuse: max normwise err %.2e, rows within %.2f of the allowed deviation\n",
              failures > failures0 ? "FAIL" : "ok", name, worst_o, worst_row);

  // step state: a step is begun once and ended once; a begin that finds the
  // pool full leaves no step behind
  {
    molot::amd::PagedKVCache st(1, 3, kNkv, kD, kPage, kv_dtype);
    const int a = st.add_sequence(), b2 = st.add_sequence();
    auto throws = [](auto&& fn) {
      try {
        fn();
      } catch (const std::runtime_error&) {
        return true;
      }
      return false;
    };
    CHECK(throws([&] { st.end_decode(); }), "%s end_decode without a step", name);
    CHECK(throws([&] { st.end_prefill(); }), "%s end_prefill without a step", name);
    st.begin_prefill(a, 30);  // 2 of the 3 blocks
    CHECK(throws([&] { st.begin_decode({a}); }), "%s begin inside a step", name);
    CHECK(throws([&] { st.end_decode(); }), "%s end_decode inside a prefill", name);
    st.end_prefill();
    CHECK(throws([&] { st.end_prefill(); }), "%s second end_prefill", name);
    CHECK(throws([&] { st.begin_prefill(b2, 20); }), "%s prefill beyond the pool", name);
    st.begin_decode({a});  // no step was left open by the failed begin
    st.end_decode();
    CHECK(st.length(a) == 31 && st.length(b2) == 0, "%s lengths after the state checks %d %d",
          name, st.length(a), st.length(b2));
  }
  // a full pool reports what a full contiguous cache does (forward.h:570)
  {
    molot::amd::PagedKVCache small(1, 2, kNkv, kD, kPage, kv_dtype);
    const int s = small.add_sequence();
    bool threw = false;
    try {
      small.begin_prefill(s, 40);
    } catch (const std::runtime_error& e) {
      threw = std::strcmp(e.what(), "fwd: KV cache full") == 0;
    }
    CHECK(threw, "%s full pool did not throw 'fwd: KV cache full'", name);
  }
  return failures - failures0;
}

}  // namespace

int main() {
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) {
    std::printf("no GPU\n");
    return 2;
  }
  run_scenario(MOLOT_KV_BF16, "bf16");
  run_scenario(MOLOT_KV_Q8, "Q8");
  std::printf(failures ? "FAILED (%d)\n" : "PASSED\n", failures);
  return failures ? 1 : 0;
}
