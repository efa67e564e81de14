// step_bench.cpp -- times forward + backward steps through the C++ op layer
// (libcandle_fused_attn.so), as a C++ caller runs them: every step calls fused_attention_qkv and
// the node's bwd, so its outputs, L and gradient are allocated per step (from the layer's memory
// pool) and the workspace is the one the node keeps. bench.py runs it beside its C-ABI step.
//
//   cfa_step_bench b h s d causal warmup steps
//
// Inputs are ~N(0, 1) (a splitmix64 stream through Box-Muller, seed fixed): the step's time does
// not depend on the values. Prints one JSON line: the mean ms per step over `steps` back-to-back
// steps after `warmup` untimed ones, timed by HIP events on the step's stream.
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "candle_fused_attn.hpp"

namespace {

uint64_t splitmix64(uint64_t& x) {
  uint64_t z = (x += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

std::vector<float> normal(std::size_t n, uint64_t seed) {
  std::vector<float> out(n);
  for (std::size_t i = 0; i < n; i += 2) {
    // Two uniforms in (0, 1], then Box-Muller.
    const double u1 = (static_cast<double>(splitmix64(seed) >> 11) + 1.0) * 0x1.0p-53;
    const double u2 = static_cast<double>(splitmix64(seed) >> 11) * 0x1.0p-53;
    const double r = std::sqrt(-2.0 * std::log(u1)), t = 6.283185307179586 * u2;
    out[i] = static_cast<float>(r * std::cos(t));
    if (i + 1 < n) out[i + 1] = static_cast<float>(r * std::sin(t));
  }
  return out;
}

void check(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    std::fprintf(stderr, "step_bench: %s: %s\n", what, hipGetErrorString(e));
    std::exit(1);
  }
}

}  // namespace

int main(int argc, char** argv) {
  namespace cfa = candle_fused_attn;
  if (argc != 8) {
    std::fprintf(stderr, "usage: %s b h s d causal warmup steps\n", argv[0]);
    return 2;
  }
  const std::size_t b = std::strtoull(argv[1], nullptr, 10), h = std::strtoull(argv[2], nullptr, 10);
  const std::size_t s = std::strtoull(argv[3], nullptr, 10), d = std::strtoull(argv[4], nullptr, 10);
  const bool causal = std::atoi(argv[5]) != 0;
  const int warmup = std::atoi(argv[6]), steps = std::atoi(argv[7]);
  if (b == 0 || h == 0 || s == 0 || d == 0 || warmup < 0 || steps <= 0) {
    std::fprintf(stderr, "step_bench: sizes and steps must be positive\n");
    return 2;
  }
  hipStream_t stream = nullptr;
  check(hipStreamCreate(&stream), "stream");
  try {
    const cfa::Tensor qkv = cfa::Tensor::from_host(normal(b * s * 3 * h * d, 0), {b, s, 3 * h * d},
                                                   stream);
    const cfa::Tensor dout = cfa::Tensor::from_host(normal(b * s * h * d, 1), {b, s, h * d}, stream);
    auto step = [&] {
      const cfa::QkvApplied r = cfa::fused_attention_qkv(qkv, h, 0.125f, causal, stream);
      const cfa::Tensor grad = r.node->bwd(r.input, r.out, dout, stream);
      (void)grad;
    };
    for (int i = 0; i < warmup; ++i) step();
    hipEvent_t e0, e1;
    check(hipEventCreate(&e0), "event");
    check(hipEventCreate(&e1), "event");
    check(hipStreamSynchronize(stream), "sync");
    check(hipEventRecord(e0, stream), "event record");
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < steps; ++i) step();
    const auto t1 = std::chrono::steady_clock::now();
    check(hipEventRecord(e1, stream), "event record");
    check(hipEventSynchronize(e1), "event sync");
    float ms = 0.0f;
    check(hipEventElapsedTime(&ms, e0, e1), "elapsed time");
    // The host's time to enqueue a step (the loop returns before the GPU is done unless the host
    // is the bottleneck).
    const double host_ms = std::chrono::duration<double, std::milli>(t1 - t0).count() / steps;
    std::printf("{\"fwd_bwd_ms\": %.5f, \"host_enqueue_ms\": %.5f, \"steps\": %d, "
                "\"warmup\": %d, \"b\": %zu, \"h\": %zu, \"s\": %zu, \"d\": %zu, "
                "\"causal\": %s}\n",
                ms / steps, host_ms, steps, warmup, b, h, s, d, causal ? "true" : "false");
    check(hipEventDestroy(e0), "event");
    check(hipEventDestroy(e1), "event");
  } catch (const cfa::Error& e) {
    std::fprintf(stderr, "step_bench: %s\n", e.what());
    return 1;
  }
  check(hipStreamDestroy(stream), "stream");
  return 0;
}
