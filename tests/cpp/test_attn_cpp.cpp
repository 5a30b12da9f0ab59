// Self-check of the header-only C++ layer (include/molot_amd/attn.hpp) on the
// GPU, in the style of the reference's own self-checking benchmark
// (bench/bench.cc:35-43: CHECK counts failures, exit status 1 on any).
// The checker is the CPU oracle (oracle/attn_oracle.c), linked as a test
// dependency.  Run by tests/test_cpp_layer.py.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <vector>

#include "attn_oracle.h"
#include "molot_amd/attn.hpp"

#include "check_util.hpp"

int main() {
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) {
    std::printf("no GPU\n");
    return 2;
  }
  molot::ThreadPool* no_pool = nullptr;  // the reference's pool: accepted, unused

  // ---- 1. DeviceKV: 64 consecutive decode steps vs the oracle's forward.h block ----
  {
    const int nq = 8, nkv = 2, d = 128, cap = 80, steps = 64;
    const float scale = 1.0f / std::sqrt((float)d);
    std::vector<float> inv(d / 2);
    molot::amd::rope_inv_freq(500000.0f, d, inv.data());
    float* inv_d = nullptr;
    molot::amd::check_hip(hipMalloc(&inv_d, inv.size() * 4), "hipMalloc");
    molot::amd::check_hip(hipMemcpy(inv_d, inv.data(), inv.size() * 4, hipMemcpyHostToDevice), "");
    molot::amd::DeviceKV kv(cap, nkv, d);
    std::vector<float> Kref((size_t)cap * nkv * d, 0.f), Vref((size_t)cap * nkv * d, 0.f);
    Rng rng(42);
    double worst = 0;
    for (int pos = 0; pos < steps; ++pos) {
      std::vector<float> q(nq * d), k(nkv * d), v(nkv * d), ao(nq * d), ao_ref(nq * d);
      rng.normal(q);
      rng.normal(k);
      rng.normal(v);
      std::vector<float> q_ref = q, k_ref = k;
      kv.decode(q.data(), k.data(), v.data(), ao.data(), nq, pos, inv_d, scale, 0);
      orc_decode_step(q_ref.data(), k_ref.data(), v.data(), Kref.data(), Vref.data(),
                      ao_ref.data(), nq, nkv, d, pos, pos, inv.data(), scale, 0, ORC_KV_F32, 1);
      worst = std::fmax(worst, normwise(ao, ao_ref));
      CHECK(normwise(q, q_ref) < 1e-6, "rotated q differs at pos %d", pos);
    }
    CHECK(kv.n == steps, "cache length %d", kv.n);
    CHECK(worst < 1e-5, "DeviceKV decode normwise err %g", worst);
    std::printf("[%s] DeviceKV %d decode steps: max normwise err %.2e\n",
                worst < 1e-5 ? "ok" : "FAIL", steps, worst);
    // the cache holds exactly what the oracle appended
    std::vector<float> Kd((size_t)steps * nkv * d);
    molot::amd::check_hip(hipMemcpy(Kd.data(), kv.k, Kd.size() * 4, hipMemcpyDeviceToHost), "");
    double kerr = 0;
    for (size_t i = 0; i < Kd.size(); ++i) kerr = std::fmax(kerr, std::fabs(Kd[i] - Kref[i]));
    CHECK(kerr < 1e-5, "appended K differs by %g", kerr);

    // ---- 1b. with the layer's norms (forward.h:554-568), gemma-style scale 1 ----
    {
      molot::amd::DeviceKV kvn(cap, nkv, d);
      std::vector<float> Kn((size_t)cap * nkv * d, 0.f), Vn((size_t)cap * nkv * d, 0.f);
      std::vector<float> qw(d), kw(d);
      rng.normal(qw);
      rng.normal(kw);
      for (int i = 0; i < d; ++i) {
        qw[i] = 1.0f + 0.2f * qw[i];
        kw[i] = 1.0f + 0.2f * kw[i];
      }
      float* w_d = nullptr;
      molot::amd::check_hip(hipMalloc(&w_d, 2 * d * 4), "hipMalloc");
      molot::amd::check_hip(hipMemcpy(w_d, qw.data(), d * 4, hipMemcpyHostToDevice), "");
      molot::amd::check_hip(hipMemcpy(w_d + d, kw.data(), d * 4, hipMemcpyHostToDevice), "");
      molot::amd::LayerNorms nm;
      nm.q_norm = w_d;
      nm.k_norm = w_d + d;
      nm.v_norm = true;
      nm.eps = 1e-6f;
      double wn = 0;
      for (int pos = 0; pos < 40; ++pos) {
        std::vector<float> q(nq * d), k(nkv * d), v(nkv * d), ao(nq * d), ao_ref(nq * d);
        rng.normal(q);
        rng.normal(k);
        rng.normal(v);
        std::vector<float> q_ref = q, k_ref = k;
        kvn.decode(q.data(), k.data(), v.data(), ao.data(), nq, pos, inv_d, 1.0f, 0, nm);
        orc_decode_step_norm(q_ref.data(), k_ref.data(), v.data(), Kn.data(), Vn.data(),
                             ao_ref.data(), nq, nkv, d, pos, pos, qw.data(), kw.data(), 1, 1e-6f,
                             inv.data(), 1.0f, 0, ORC_KV_F32, 1);
        wn = std::fmax(wn, normwise(ao, ao_ref));
        CHECK(normwise(q, q_ref) < 2e-6, "normed rotated q differs at pos %d", pos);
      }
      CHECK(wn < 1e-5, "DeviceKV decode with norms normwise err %g", wn);
      std::printf("[%s] DeviceKV 40 decode steps with q/k/v norms: max normwise err %.2e\n",
                  wn < 1e-5 ? "ok" : "FAIL", wn);
      (void)hipFree(w_d);
    }

    // ---- 1c. a Q8 cache (rows quantized as quant.h:34-50) ----
    // Each step's appended k and v rows against the oracle's quantizer (the
    // rotated k may differ by an fp32 ulp before quantization: codes within
    // one, scales within an ulp), then the GPU's bytes replace the oracle's
    // so the attention is compared on identical caches.
    {
      const int R = orc_q8_row_bytes(nkv, d);
      molot::amd::DeviceKV kvq(cap, nkv, d, MOLOT_KV_Q8);
      std::vector<uint8_t> Kq((size_t)cap * R, 0), Vq((size_t)cap * R, 0), row(R);
      double wq = 0, sdiff = 0;
      int cdiff = 0;
      for (int pos = 0; pos < 48; ++pos) {
        std::vector<float> q(nq * d), k(nkv * d), v(nkv * d), ao(nq * d), ao_ref(nq * d);
        rng.normal(q);
        rng.normal(k);
        rng.normal(v);
        std::vector<float> q_ref = q, k_ref = k;
        kvq.decode(q.data(), k.data(), v.data(), ao.data(), nq, pos, inv_d, scale, 0);
        orc_decode_step(q_ref.data(), k_ref.data(), v.data(), Kq.data(), Vq.data(),
                        ao_ref.data(), nq, nkv, d, pos, pos, inv.data(), scale, 0, ORC_KV_Q8, 1);
        for (int side = 0; side < 2; ++side) {
          std::vector<uint8_t>& C = side ? Vq : Kq;
          const char* src = (const char*)(side ? kvq.v : kvq.k) + (size_t)pos * R;
          molot::amd::check_hip(hipMemcpy(row.data(), src, R, hipMemcpyDeviceToHost), "D2H row");
          uint8_t* ref_row = C.data() + (size_t)pos * R;
          for (int i = 0; i < nkv * d; ++i)
            cdiff = std::max(cdiff, std::abs((int)(int8_t)row[i] - (int)(int8_t)ref_row[i]));
          for (int h = 0; h < nkv; ++h) {
            float a, b;
            std::memcpy(&a, row.data() + nkv * d + 4 * h, 4);
            std::memcpy(&b, ref_row + nkv * d + 4 * h, 4);
            sdiff = std::fmax(sdiff, std::fabs(a - b) / b);
          }
          std::memcpy(ref_row, row.data(), R);
        }
        std::vector<float> o2(nq * d);
        orc_attn_decode(q_ref.data(), Kq.data(), Vq.data(), o2.data(), nq, nkv, pos + 1, d, scale,
                        pos, 0, ORC_KV_Q8, 0, 0, 0, nullptr, 0, 1);
        wq = std::fmax(wq, normwise(ao, o2));
        CHECK(normwise(q, q_ref) < 1e-6, "Q8: rotated q differs at pos %d", pos);
      }
      CHECK(cdiff <= 1 && sdiff <= 1e-6, "Q8 appended rows: codes off by %d, scales by %g", cdiff,
            sdiff);
      CHECK(wq < 1e-5, "DeviceKV Q8 decode normwise err %g", wq);
      std::printf("[%s] DeviceKV Q8 48 decode steps: max normwise err %.2e, appended codes "
                  "within %d\n",
                  (wq < 1e-5 && cdiff <= 1 && sdiff <= 1e-6) ? "ok" : "FAIL", wq, cdiff);
    }

    // ---- 1d. a layer without RoPE, and a layer reading this cache (shared KV) ----
    {
      molot::amd::DeviceKV kvn(cap, nkv, d);
      std::vector<float> Kn((size_t)cap * nkv * d, 0.f), Vn((size_t)cap * nkv * d, 0.f);
      double wn = 0, ws = 0;
      for (int pos = 0; pos < 40; ++pos) {
        std::vector<float> q(nq * d), k(nkv * d), v(nkv * d), ao(nq * d), ao_ref(nq * d);
        rng.normal(q);
        rng.normal(k);
        rng.normal(v);
        std::vector<float> q_ref = q, k_ref = k;
        kvn.decode(q.data(), k.data(), v.data(), ao.data(), nq, pos, nullptr, scale, 0);
        orc_decode_step(q_ref.data(), k_ref.data(), v.data(), Kn.data(), Vn.data(), ao_ref.data(),
                        nq, nkv, d, pos, pos, nullptr, scale, 0, ORC_KV_F32, 1);
        wn = std::fmax(wn, normwise(ao, ao_ref));
        CHECK(q == q_ref, "NoPE decode rotated q at pos %d", pos);
        // a shared-KV layer over the same cache, with RoPE
        std::vector<float> q2(nq * d), ao2(nq * d), ao2_ref(nq * d);
        rng.normal(q2);
        std::vector<float> q2_ref = q2;
        kvn.decode_shared(q2.data(), ao2.data(), nq, pos, inv_d, scale, 0);
        orc_decode_step_shared(q2_ref.data(), Kn.data(), Vn.data(), ao2_ref.data(), nq, nkv, d,
                               pos + 1, pos, nullptr, 0.f, inv.data(), scale, 0, ORC_KV_F32, 1);
        ws = std::fmax(ws, normwise(ao2, ao2_ref));
        CHECK(normwise(q2, q2_ref) < 1e-6, "shared decode q at pos %d", pos);
      }
      CHECK(wn < 1e-5, "DeviceKV NoPE decode normwise err %g", wn);
      CHECK(ws < 1e-5, "DeviceKV shared decode normwise err %g", ws);
      std::printf("[%s] DeviceKV NoPE decode and shared-KV decode, 40 steps: %.2e, %.2e\n",
                  (wn < 1e-5 && ws < 1e-5) ? "ok" : "FAIL", wn, ws);
    }

    // ---- 2. attn.h drop-in on the same cache, host q/o, sliding window ----
    std::vector<float> q(nq * d), o(nq * d), o_ref(nq * d);
    rng.normal(q);
    molot::amd::attn_decode_gqa_cache(q.data(), (const float*)kv.k, (const float*)kv.v, o.data(),
                                      nq, nkv, kv.n, d, scale, kv.n - 1, 17, *no_pool);
    orc_attn_decode_gqa_cache(q.data(), Kref.data(), Vref.data(), o_ref.data(), nq, nkv, kv.n, d,
                              scale, kv.n - 1, 17, 1);
    const double e2 = normwise(o, o_ref);
    CHECK(e2 < 1e-5, "attn_decode_gqa_cache drop-in err %g", e2);
    std::printf("[%s] attn_decode_gqa_cache drop-in (window 17): err %.2e\n",
                e2 < 1e-5 ? "ok" : "FAIL", e2);

    // ---- 3. cache full throws, as forward.h:570 ----
    bool threw = false;
    molot::amd::DeviceKV small(1, nkv, d);
    std::vector<float> qq(nq * d, 0.1f), kk(nkv * d, 0.2f), vv(nkv * d, 0.3f), oo(nq * d);
    small.decode(qq.data(), kk.data(), vv.data(), oo.data(), nq, 0, inv_d, scale, 0);
    try {
      small.decode(qq.data(), kk.data(), vv.data(), oo.data(), nq, 1, inv_d, scale, 0);
    } catch (const std::runtime_error& e) {
      threw = std::string(e.what()).find("KV cache full") != std::string::npos;
    }
    CHECK(threw, "second append into a 1-slot cache did not throw");
    // one token attends only to itself: o = v
    double e3 = 0;
    for (int h = 0; h < nq; ++h)
      for (int j = 0; j < d; ++j) e3 = std::fmax(e3, std::fabs(oo[h * d + j] - 0.3f));
    CHECK(e3 < 1e-6, "single-token attention err %g", e3);
    std::printf("[%s] cache-full error and single-token output\n", threw && e3 < 1e-6 ? "ok" : "FAIL");
    (void)hipFree(inv_d);
  }

  // ---- 5. host vectors whose sizes are not multiples of 4 floats (3 q heads
  // and 1 KV head of d = 34: 102 and 34 floats), staged through the pinned
  // mirror on 16-byte slots; then the same step with q and ao on the device
  // and k, v on the host (a mixed call) ----
  {
    const int nq = 3, nkv = 1, d = 34, cap = 24, steps = 20;
    const float scale = 1.0f / std::sqrt((float)d);
    std::vector<float> inv(d / 2);
    molot::amd::rope_inv_freq(10000.0f, d, inv.data());
    float* inv_d = nullptr;
    molot::amd::check_hip(hipMalloc(&inv_d, inv.size() * 4), "hipMalloc");
    molot::amd::check_hip(hipMemcpy(inv_d, inv.data(), inv.size() * 4, hipMemcpyHostToDevice), "");
    molot::amd::DeviceKV kv(cap, nkv, d);
    std::vector<float> Kref((size_t)cap * nkv * d, 0.f), Vref((size_t)cap * nkv * d, 0.f);
    Rng rng(7);
    double worst = 0, qworst = 0;
    float *q_dev = nullptr, *ao_dev = nullptr;
    molot::amd::check_hip(hipMalloc(&q_dev, nq * d * 4), "hipMalloc");
    molot::amd::check_hip(hipMalloc(&ao_dev, nq * d * 4), "hipMalloc");
    for (int pos = 0; pos < steps; ++pos) {
      std::vector<float> q(nq * d), k(nkv * d), v(nkv * d), ao(nq * d), ao_ref(nq * d);
      rng.normal(q);
      rng.normal(k);
      rng.normal(v);
      std::vector<float> q_ref = q, k_ref = k;
      if (pos % 2 == 0) {
        kv.decode(q.data(), k.data(), v.data(), ao.data(), nq, pos, inv_d, scale, 0);
      } else {
        molot::amd::check_hip(hipMemcpy(q_dev, q.data(), nq * d * 4, hipMemcpyHostToDevice), "");
        kv.decode(q_dev, k.data(), v.data(), ao_dev, nq, pos, inv_d, scale, 0);
        molot::amd::check_hip(hipMemcpy(q.data(), q_dev, nq * d * 4, hipMemcpyDeviceToHost), "");
        molot::amd::check_hip(hipMemcpy(ao.data(), ao_dev, nq * d * 4, hipMemcpyDeviceToHost), "");
      }
      orc_decode_step(q_ref.data(), k_ref.data(), v.data(), Kref.data(), Vref.data(),
                      ao_ref.data(), nq, nkv, d, pos, pos, inv.data(), scale, 0, ORC_KV_F32, 1);
      worst = std::fmax(worst, normwise(ao, ao_ref));
      qworst = std::fmax(qworst, normwise(q, q_ref));
    }
    CHECK(worst < 1e-5, "d = 34 host/device decode normwise err %g", worst);
    CHECK(qworst < 1e-6, "d = 34 rotated q err %g", qworst);
    std::printf("[%s] DeviceKV 3q/1kv/d34, host and mixed pointers, %d steps: %.2e (q %.2e)\n",
                worst < 1e-5 && qworst < 1e-6 ? "ok" : "FAIL", steps, worst, qworst);
    (void)hipFree(q_dev);
    (void)hipFree(ao_dev);
    (void)hipFree(inv_d);
  }

  // ---- 4. an unsupported (odd) head dim surfaces as std::runtime_error ----
  {
    bool threw = false;
    try {
      float* dq = nullptr;
      molot::amd::check_hip(hipMalloc(&dq, 4 * 96 * 4), "");
      molot::amd::attn_decode_gqa_cache(dq, dq, dq, dq, 4, 4, 1, 95, 0.1f, 0, 0, *no_pool);
    } catch (const std::runtime_error& e) {
      threw = std::string(e.what()).find("unsupported") != std::string::npos;
    }
    CHECK(threw, "head dim 95 did not raise");
    std::printf("[%s] unsupported head dim raises\n", threw ? "ok" : "FAIL");
  }

  std::printf("%s (%d failures)\n", failures ? "FAILED" : "PASSED", failures);
  return failures ? 1 : 0;
}
