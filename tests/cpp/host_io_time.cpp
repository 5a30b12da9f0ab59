// Time of one synchronous decode-layer call through the C++ drop-in
// (include/molot_amd/attn.hpp, DeviceKV::decode: forward.h:556-591) with the
// reference's host vectors (q, k_new, v_new, ao staged through the pinned
// mirror) against the same call with device vectors.  Usage:
//   host_io_time nq nkv d n window [calls] [layers]
// Each call appends at slot n (the cache length is reset before it) and
// attends n + 1 rows (the last `window` of them if window > 0), fp32 KV;
// `layers` caches are cycled so that the stream is not served from the
// Infinity Cache.  Prints one line:
//   host_us=<us per call> device_us=<us per call> calls=<calls> layers=<layers>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <memory>
#include <vector>

#include "molot_amd/attn.hpp"

int main(int argc, char** argv) {
  if (argc < 6) {
    std::fprintf(stderr, "usage: %s nq nkv d n window [calls] [layers]\n", argv[0]);
    return 2;
  }
  const int nq = std::atoi(argv[1]), nkv = std::atoi(argv[2]), d = std::atoi(argv[3]);
  const int n = std::atoi(argv[4]), window = std::atoi(argv[5]);
  const int calls = argc > 6 ? std::atoi(argv[6]) : 200;
  const int layers = argc > 7 ? std::atoi(argv[7]) : 8;
  using molot::amd::check_hip;
  std::vector<std::unique_ptr<molot::amd::DeviceKV>> kv;
  for (int l = 0; l < layers; ++l) {
    kv.emplace_back(new molot::amd::DeviceKV(n + 1, nkv, d));
    const size_t bytes = (size_t)(n + 1) * nkv * d * sizeof(float);
    check_hip(hipMemset(kv.back()->k, 0, bytes), "hipMemset");
    check_hip(hipMemset(kv.back()->v, 0, bytes), "hipMemset");
  }
  std::vector<float> inv(d / 2);
  molot::amd::rope_inv_freq(500000.0f, d, inv.data());
  float* inv_d = nullptr;
  check_hip(hipMalloc(&inv_d, inv.size() * 4), "hipMalloc");
  check_hip(hipMemcpy(inv_d, inv.data(), inv.size() * 4, hipMemcpyHostToDevice), "H2D");
  std::vector<float> q(nq * d, 0.01f), k(nkv * d, 0.02f), v(nkv * d, 0.03f), ao(nq * d);
  float *qd = nullptr, *kd = nullptr, *vd = nullptr, *aod = nullptr;
  check_hip(hipMalloc(&qd, q.size() * 4), "hipMalloc");
  check_hip(hipMalloc(&kd, k.size() * 4), "hipMalloc");
  check_hip(hipMalloc(&vd, v.size() * 4), "hipMalloc");
  check_hip(hipMalloc(&aod, ao.size() * 4), "hipMalloc");
  check_hip(hipDeviceSynchronize(), "sync");
  const float scale = 1.0f / std::sqrt((float)d);
  auto run = [&](bool host, int count) {
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < count; ++i) {
      molot::amd::DeviceKV& c = *kv[i % layers];
      c.n = n;
      if (host)
        c.decode(q.data(), k.data(), v.data(), ao.data(), nq, n, inv_d, scale, window);
      else
        c.decode(qd, kd, vd, aod, nq, n, inv_d, scale, window);
    }
    const auto t1 = std::chrono::steady_clock::now();
    return std::chrono::duration<double, std::micro>(t1 - t0).count() / count;
  };
  run(true, 10);
  run(false, 10);
  const double host_us = run(true, calls);
  const double dev_us = run(false, calls);
  std::printf("host_us=%.2f device_us=%.2f calls=%d layers=%d\n", host_us, dev_us, calls, layers);
  return 0;
}
