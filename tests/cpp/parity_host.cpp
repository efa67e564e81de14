// parity_host.cpp -- the reference's integration tests (tests/parity.rs) for the C++ op layer
// (candle-fused-attn_amd/host/candle_fused_attn.hpp), plus the layer's own views, copy fallbacks
// and errors.
//
// The reference checks both entry points against a composed attention on candle's CPU
// (tests/parity.rs:53-80, :147-170); here the checker is the CPU oracle (oracle/liboracle.so, a
// restatement of that composed path in C) in fp32, and in fp64 for the spread. Inputs are the
// reference's closed-form sequences (tests/parity.rs:129-145): x_i = 1.5 sin(0.618034 i),
// w_i = cos(0.414213 i), so no generator is involved.
//
// Usage: parity_host --cpu | --gpu [--only NAME]. --cpu runs what needs no device (views,
// predicates, errors raised before any launch, empty inputs); --gpu runs the parity cases on
// device 0. Exit status 0 when every selected case passed.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "candle_fused_attn.hpp"

extern "C" {
int oracle_forward_f32(const float* q, const float* k, const float* v, int64_t b, int64_t h,
                       int64_t s, int64_t d, float scale, int causal, float* o, float* l,
                       int threads);
int oracle_backward_f32(const float* q, const float* k, const float* v, const float* o,
                        const float* l, const float* d_o, int64_t b, int64_t h, int64_t s,
                        int64_t d, float scale, int causal, float* dq, float* dk, float* dv,
                        int threads);
int oracle_forward_f64(const double* q, const double* k, const double* v, int64_t b, int64_t h,
                       int64_t s, int64_t d, double scale, int causal, double* o, double* l,
                       int threads);
int oracle_backward_f64(const double* q, const double* k, const double* v, const double* o,
                        const double* l, const double* d_o, int64_t b, int64_t h, int64_t s,
                        int64_t d, double scale, int causal, double* dq, double* dk, double* dv,
                        int threads);
}

namespace cfa = candle_fused_attn;
using Dims = std::vector<std::size_t>;

namespace {

struct Failure {
  std::string what;
};

void expect(bool ok, const std::string& what) {
  if (!ok) throw Failure{what};
}

// The call must throw cfa::Error whose message contains `needle`.
void expect_error(const std::function<void()>& f, const std::string& needle) {
  try {
    f();
  } catch (const cfa::Error& e) {
    expect(std::string(e.what()).find(needle) != std::string::npos,
           "error \"" + std::string(e.what()) + "\" lacks \"" + needle + "\"");
    return;
  }
  throw Failure{"no error; expected one containing \"" + needle + "\""};
}

hipStream_t g_stream = nullptr;

// tests/parity.rs:129-145: the projection and the loss weights.
struct Inputs {
  std::size_t b, s, h, d;
  std::vector<float> x;  // [b, s, 3 h d]
  std::vector<float> w;  // [b, s, h d]
};

Inputs inputs(std::size_t b, std::size_t s, std::size_t h, std::size_t d) {
  Inputs in{b, s, h, d, std::vector<float>(b * s * 3 * h * d), std::vector<float>(b * s * h * d)};
  for (std::size_t i = 0; i < in.x.size(); ++i) {
    in.x[i] = std::sin(static_cast<float>(i) * 0.618034f) * 1.5f;
  }
  for (std::size_t i = 0; i < in.w.size(); ++i) {
    in.w[i] = std::cos(static_cast<float>(i) * 0.414213f);
  }
  return in;
}

// part p (0 q, 1 k, 2 v) of the projection as contiguous [b, h, s, d].
template <typename T>
std::vector<T> head_split(const Inputs& in, int p) {
  const std::size_t b = in.b, s = in.s, h = in.h, d = in.d;
  std::vector<T> out(b * h * s * d);
  for (std::size_t ib = 0; ib < b; ++ib)
    for (std::size_t ih = 0; ih < h; ++ih)
      for (std::size_t is = 0; is < s; ++is)
        for (std::size_t c = 0; c < d; ++c)
          out[((ib * h + ih) * s + is) * d + c] =
              in.x[(ib * s + is) * 3 * h * d + p * h * d + ih * d + c];
  return out;
}

// The loss weights as the output gradient, contiguous [b, h, s, d].
template <typename T>
std::vector<T> weights_bhsd(const Inputs& in) {
  const std::size_t b = in.b, s = in.s, h = in.h, d = in.d;
  std::vector<T> out(b * h * s * d);
  for (std::size_t ib = 0; ib < b; ++ib)
    for (std::size_t ih = 0; ih < h; ++ih)
      for (std::size_t is = 0; is < s; ++is)
        for (std::size_t c = 0; c < d; ++c)
          out[((ib * h + ih) * s + is) * d + c] = in.w[(ib * s + is) * h * d + ih * d + c];
  return out;
}

// The oracle's output O, L, dQ, dK, dV ([b, h, s, d] / [b, h, s]) in precision T.
template <typename T>
struct Ref {
  std::vector<T> o, l, dq, dk, dv;
};

template <typename T>
Ref<T> oracle(const Inputs& in, T scale, bool causal) {
  const auto q = head_split<T>(in, 0), k = head_split<T>(in, 1), v = head_split<T>(in, 2);
  const auto g = weights_bhsd<T>(in);
  const int64_t b = in.b, h = in.h, s = in.s, d = in.d;
  Ref<T> r{std::vector<T>(q.size()), std::vector<T>(b * h * s), std::vector<T>(q.size()),
           std::vector<T>(q.size()), std::vector<T>(q.size())};
  int rc;
  if constexpr (sizeof(T) == 4) {
    rc = oracle_forward_f32(q.data(), k.data(), v.data(), b, h, s, d, scale, causal, r.o.data(),
                            r.l.data(), 8);
    rc |= oracle_backward_f32(q.data(), k.data(), v.data(), r.o.data(), r.l.data(), g.data(), b,
                              h, s, d, scale, causal, r.dq.data(), r.dk.data(), r.dv.data(), 8);
  } else {
    rc = oracle_forward_f64(q.data(), k.data(), v.data(), b, h, s, d, scale, causal, r.o.data(),
                            r.l.data(), 8);
    rc |= oracle_backward_f64(q.data(), k.data(), v.data(), r.o.data(), r.l.data(), g.data(), b,
                              h, s, d, scale, causal, r.dq.data(), r.dk.data(), r.dv.data(), 8);
  }
  expect(rc == 0, "oracle failed");
  return r;
}

template <typename T>
double max_abs(const std::vector<float>& a, const std::vector<T>& r) {
  expect(a.size() == r.size(), "size mismatch: " + std::to_string(a.size()) + " vs " +
                                   std::to_string(r.size()));
  double m = 0;
  for (std::size_t i = 0; i < a.size(); ++i) {
    const double e = std::fabs(static_cast<double>(a[i]) - static_cast<double>(r[i]));
    if (!(e <= m)) m = e;  // a NaN stays NaN
  }
  return m;
}

// Max |a - r| / max(1, |r|): L is a log-sum-exp of size up to |scale q.k| + ln s, so its error
// is measured relative to its magnitude (absolute below 1).
double max_rel1(const std::vector<float>& a, const std::vector<float>& r) {
  expect(a.size() == r.size(), "size mismatch");
  double m = 0;
  for (std::size_t i = 0; i < a.size(); ++i) {
    const double e = std::fabs(static_cast<double>(a[i]) - static_cast<double>(r[i])) /
                     std::max(1.0, std::fabs(static_cast<double>(r[i])));
    if (!(e <= m)) m = e;
  }
  return m;
}

// Normwise relative error ||a - r|| / ||r|| (Frobenius norms, in double).
template <typename A, typename R>
double rel_fro(const std::vector<A>& a, const std::vector<R>& r) {
  expect(a.size() == r.size(), "size mismatch");
  double num = 0, den = 0;
  for (std::size_t i = 0; i < a.size(); ++i) {
    const double x = static_cast<double>(r[i]), e = static_cast<double>(a[i]) - x;
    num += e * e;
    den += x * x;
  }
  return den > 0 ? std::sqrt(num / den) : std::sqrt(num);
}

bool bit_equal(const std::vector<float>& a, const std::vector<float>& b) {
  return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * sizeof(float)) == 0;
}

// [b, h, s, d] host values of a merged [b, s, h d] tensor's values.
std::vector<float> merged_to_bhsd(const std::vector<float>& m, const Inputs& in, std::size_t part,
                                  std::size_t parts) {
  const std::size_t b = in.b, s = in.s, h = in.h, d = in.d;
  std::vector<float> out(b * h * s * d);
  for (std::size_t ib = 0; ib < b; ++ib)
    for (std::size_t ih = 0; ih < h; ++ih)
      for (std::size_t is = 0; is < s; ++is)
        for (std::size_t c = 0; c < d; ++c)
          out[((ib * h + ih) * s + is) * d + c] =
              m[(ib * s + is) * parts * h * d + part * h * d + ih * d + c];
  return out;
}

// q, k, v as [b, h, s, d] views of the projection (tests/parity.rs:38-50 builds them with
// narrow + reshape + transpose; candle's reshape copies the narrowed, non-contiguous part, while
// these views read the projection in place, strides [s 3hd, d, 3hd, 1], so the kernels' strided
// path is the one exercised).
std::array<cfa::Tensor, 3> qkv_views(const cfa::Tensor& qkv, std::size_t h, std::size_t d) {
  const cfa::Layout& l = qkv.layout();
  const std::size_t b = l.shape[0], s = l.shape[1];
  auto split = [&](std::size_t i) {
    return cfa::Tensor(qkv.storage(),
                       cfa::Layout{l.start_offset + i * h * d, {b, h, s, d},
                                   {l.stride[0], d, l.stride[1], l.stride[2]}});
  };
  return {split(0), split(1), split(2)};
}

// One forward + backward of `path` (0: fused_attention on the views, 1: fused_attention_qkv),
// results in [b, h, s, d] host order: O, L, dQ, dK, dV.
struct Run {
  std::vector<float> o, l, dq, dk, dv;
};

Run run(int path, const Inputs& in, bool causal) {
  const std::size_t b = in.b, s = in.s, h = in.h, d = in.d;
  const float scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(d)));
  const cfa::Tensor qkv = cfa::Tensor::from_host(in.x, {b, s, 3 * h * d}, g_stream);
  Run r;
  if (path == 0) {
    const auto [q, k, v] = qkv_views(qkv, h, d);
    const cfa::Applied a = cfa::fused_attention(q, k, v, scale, causal, g_stream);
    // The gradient of sum(out o w) with respect to the raw [b, s, h, d] output is w itself.
    const cfa::Tensor g = cfa::Tensor::from_host(in.w, {b, s, h, d}, g_stream);
    const auto grads = a.node->bwd(a.q, a.k, a.v, a.raw, g, g_stream);
    r.o = a.out.to_host(g_stream);
    r.l = a.node->saved_lse().to_host(g_stream);
    r.dq = grads[0].to_host(g_stream);
    r.dk = grads[1].to_host(g_stream);
    r.dv = grads[2].to_host(g_stream);
  } else {
    const cfa::QkvApplied a = cfa::fused_attention_qkv(qkv, h, scale, causal, g_stream);
    const cfa::Tensor g = cfa::Tensor::from_host(in.w, {b, s, h * d}, g_stream);
    const cfa::Tensor dqkv = a.node->bwd(a.input, a.out, g, g_stream);
    r.o = merged_to_bhsd(a.out.to_host(g_stream), in, 0, 1);
    r.l = a.node->saved_lse().to_host(g_stream);
    const auto all = dqkv.to_host(g_stream);
    r.dq = merged_to_bhsd(all, in, 0, 3);
    r.dk = merged_to_bhsd(all, in, 1, 3);
    r.dv = merged_to_bhsd(all, in, 2, 3);
  }
  return r;
}

const char* path_name(int path) { return path == 0 ? "Fused" : "FusedQkv"; }

// tests/parity.rs:147-170: every path against the fp32 oracle at `band` (max-abs on O and the
// gradients, max_rel1 on L, which the reference does not test); the fp32 oracle's own distance
// from fp64 printed beside it (the reference's "null band"). Then against fp64, normwise: O, dQ,
// dK and dV each within max(2e-6, 1.5 x the fp32 oracle's own normwise error) -- on these
// closed-form inputs the gradient is ill-conditioned, and the reference's own arithmetic in fp32
// misses 2e-6 on dQ, so the bar is to be no less accurate than it.
void check(std::size_t b, std::size_t s, std::size_t h, std::size_t d, bool causal, double band) {
  const Inputs in = inputs(b, s, h, d);
  const double scale = 1.0 / std::sqrt(static_cast<double>(d));
  const Ref<float> r32 = oracle<float>(in, static_cast<float>(scale), causal);
  const Ref<double> r64 = oracle<double>(in, scale, causal);
  const double null_o = max_abs(r32.o, r64.o);
  const double null_g = std::max({max_abs(r32.dq, r64.dq), max_abs(r32.dk, r64.dk),
                                  max_abs(r32.dv, r64.dv)});
  for (int path : {0, 1}) {
    const Run g = run(path, in, causal);
    const double eo = max_abs(g.o, r32.o);
    const double eg = std::max({max_abs(g.dq, r32.dq), max_abs(g.dk, r32.dk),
                                max_abs(g.dv, r32.dv)});
    const double el = max_rel1(g.l, r32.l);
    const double eo64 = max_abs(g.o, r64.o);
    const double eg64 = std::max({max_abs(g.dq, r64.dq), max_abs(g.dk, r64.dk),
                                  max_abs(g.dv, r64.dv)});
    std::printf("  %s b%zu s%zu h%zu d%zu causal=%d: out %.2e grad %.2e L(rel) %.2e | fp64 out %.2e "
                "grad %.2e | oracle fp32-fp64 out %.2e grad %.2e\n",
                path_name(path), b, s, h, d, causal ? 1 : 0, eo, eg, el, eo64, eg64, null_o,
                null_g);
    expect(eo < band && eg < band && el < band,
           std::string(path_name(path)) + " mismatch: out " + std::to_string(eo) + ", grad " +
               std::to_string(eg) + ", L " + std::to_string(el));
    const std::vector<float>* got[4] = {&g.o, &g.dq, &g.dk, &g.dv};
    const std::vector<float>* f32[4] = {&r32.o, &r32.dq, &r32.dk, &r32.dv};
    const std::vector<double>* f64[4] = {&r64.o, &r64.dq, &r64.dk, &r64.dv};
    const char* names[4] = {"out", "dq", "dk", "dv"};
    std::printf("    normwise vs fp64 (bar):");
    for (int i = 0; i < 4; ++i) {
      const double e = rel_fro(*got[i], *f64[i]);
      const double bar = std::max(2e-6, 1.5 * rel_fro(*f32[i], *f64[i]));
      std::printf(" %s %.2e (%.2e)", names[i], e, bar);
      expect(e <= bar, std::string(path_name(path)) + " " + names[i] + " normwise " +
                           std::to_string(e) + " > " + std::to_string(bar));
    }
    std::printf("\n");
  }
}

// --- GPU cases -----------------------------------------------------------------------------------

// tests/parity.rs:209-220 (cuda_matches_cpu), band 5e-6.
void gpu_matches_oracle() {
  for (bool causal : {false, true}) {
    for (const auto& sh : {Dims{2, 7, 3, 64}, Dims{2, 240, 6, 64}, Dims{1, 97, 2, 64}}) {
      check(sh[0], sh[1], sh[2], sh[3], causal, 5e-6);
    }
  }
}

// The other head dims the kernels take (32, 128), same band.
void gpu_other_head_dims() {
  for (bool causal : {false, true}) {
    check(2, 70, 3, 32, causal, 5e-6);
    check(1, 97, 2, 128, causal, 5e-6);
  }
}

// tests/parity.rs:172-188 at d 64 (the reference's d 8 runs on its CPU path only).
void outputs_are_merge_heads_ready() {
  const Inputs in = inputs(2, 5, 3, 64);
  const cfa::Tensor qkv = cfa::Tensor::from_host(in.x, {2, 5, 3 * 3 * 64}, g_stream);
  const auto [q, k, v] = qkv_views(qkv, 3, 64);
  const cfa::Applied a = cfa::fused_attention(q, k, v, 0.3f, false, g_stream);
  expect(a.out.dims() == Dims({2, 3, 5, 64}), "fused_attention: dims");
  expect(a.out.transpose(1, 2).is_contiguous(), "O is physically [b, s, h, d]");
  expect(a.q.storage() == qkv.storage() && a.k.storage() == qkv.storage(),
         "the views are read in place");
  const cfa::QkvApplied m = cfa::fused_attention_qkv(qkv, 3, 0.3f, false, g_stream);
  expect(m.out.dims() == Dims({2, 5, 3 * 64}), "fused_attention_qkv: dims");
  expect(m.out.is_contiguous(), "fused_attention_qkv: contiguous");
  expect(m.input.storage() == qkv.storage(), "the projection is read in place");
  // The two entry points give the same output bit for bit on the same projection.
  expect(bit_equal(a.out.transpose(1, 2).reshape({2, 5, 3 * 64}, g_stream).to_host(g_stream),
                   m.out.to_host(g_stream)),
         "fused_attention and fused_attention_qkv differ");
}

// tests/parity.rs:190-205: the saved L is read, not consumed.
void backward_twice_over_one_graph() {
  const Inputs in = inputs(1, 9, 2, 64);
  const cfa::Tensor qkv = cfa::Tensor::from_host(in.x, {1, 9, 3 * 2 * 64}, g_stream);
  const cfa::Tensor w = cfa::Tensor::from_host(in.w, {1, 9, 2 * 64}, g_stream);
  const cfa::QkvApplied a = cfa::fused_attention_qkv(qkv, 2, 0.125f, false, g_stream);
  const auto g1 = a.node->bwd(a.input, a.out, w, g_stream).to_host(g_stream);
  const auto g2 = a.node->bwd(a.input, a.out, w, g_stream).to_host(g_stream);
  expect(bit_equal(g1, g2), "FusedQkv: second backward differs");
  const auto [q, k, v] = qkv_views(qkv, 2, 64);
  const cfa::Applied f = cfa::fused_attention(q, k, v, 0.125f, true, g_stream);
  const cfa::Tensor wr = w.reshape({1, 9, 2, 64}, g_stream);
  const auto h1 = f.node->bwd(f.q, f.k, f.v, f.raw, wr, g_stream);
  const auto h2 = f.node->bwd(f.q, f.k, f.v, f.raw, wr, g_stream);
  for (int i = 0; i < 3; ++i) {
    expect(bit_equal(h1[i].to_host(g_stream), h2[i].to_host(g_stream)),
           "Fused: second backward differs in gradient " + std::to_string(i));
  }
}

// tests/parity.rs:222-241: eight reruns bit-identical, causal and not, both paths.
void backward_is_deterministic() {
  const Inputs in = inputs(4, 240, 6, 64);
  for (bool causal : {false, true}) {
    for (int path : {0, 1}) {
      const Run first = run(path, in, causal);
      for (int rerun = 0; rerun < 8; ++rerun) {
        const Run again = run(path, in, causal);
        expect(bit_equal(first.dq, again.dq) && bit_equal(first.dk, again.dk) &&
                   bit_equal(first.dv, again.dv) && bit_equal(first.o, again.o),
               std::string(path_name(path)) + ", causal " + std::to_string(causal) +
                   ": rerun " + std::to_string(rerun) + " differs from the first");
      }
    }
  }
}

// The layer's block cache: storage given back is reused for the next storage of that size on the
// stream (a step in the steady state takes no new memory), release_cached_blocks gives it back,
// and runs after a release take new blocks and give the same bits.
void cached_blocks_are_reused_and_released() {
  const Inputs in = inputs(2, 97, 3, 64);
  const Run first = run(1, in, false);
  (void)hipStreamSynchronize(g_stream);
  const std::size_t released = cfa::release_cached_blocks();
  expect(released > 0, "a run's freed storage was not cached");
  const Run again = run(1, in, false);
  expect(bit_equal(first.o, again.o) && bit_equal(first.dq, again.dq) &&
             bit_equal(first.dk, again.dk) && bit_equal(first.dv, again.dv),
         "a run after release_cached_blocks differs");
  float* a = nullptr;
  {
    const cfa::Tensor t = cfa::Tensor::empty({1000}, g_stream);
    a = t.storage_ptr();
  }
  const cfa::Tensor t2 = cfa::Tensor::empty({1000}, g_stream);
  expect(t2.storage_ptr() == a, "a freed block of the same size on the stream was not reused");
  const cfa::Tensor t3 = cfa::Tensor::empty({1000}, g_stream);
  expect(t3.storage_ptr() != a, "a block in use was handed out twice");
}

// Copy fallbacks (src/lib.rs:110-118, :163-178, :368-380): operands and a gradient the kernels
// cannot read in place are copied, and the results equal those of aligned operands bit for bit.
void copy_fallbacks_match_aligned_operands() {
  const std::size_t b = 2, s = 33, h = 2, d = 64, n = b * s * 3 * h * d;
  const Inputs in = inputs(b, s, h, d);
  // The projection at element offset 1 of a larger buffer: not float4-aligned.
  std::vector<float> shifted(n + 1, 0.0f);
  std::copy(in.x.begin(), in.x.end(), shifted.begin() + 1);
  const cfa::Tensor big = cfa::Tensor::from_host(shifted, {n + 1}, g_stream);
  const cfa::Tensor odd(big.storage(), cfa::Layout{1, {b, s, 3 * h * d}, {s * 3 * h * d, 3 * h * d, 1}});
  const cfa::Tensor qkv = cfa::Tensor::from_host(in.x, {b, s, 3 * h * d}, g_stream);
  const cfa::QkvApplied a = cfa::fused_attention_qkv(qkv, h, 0.125f, true, g_stream);
  const cfa::QkvApplied m = cfa::fused_attention_qkv(odd, h, 0.125f, true, g_stream);
  expect(m.input.storage() != odd.storage() && m.input.layout().start_offset == 0,
         "a misaligned projection is copied to offset 0");
  expect(bit_equal(a.out.to_host(g_stream), m.out.to_host(g_stream)), "qkv copy: outputs differ");
  // A gradient at offset 1: copied before the backward.
  std::vector<float> wshift(in.w.size() + 1, 0.0f);
  std::copy(in.w.begin(), in.w.end(), wshift.begin() + 1);
  const cfa::Tensor wbig = cfa::Tensor::from_host(wshift, {wshift.size()}, g_stream);
  const cfa::Tensor wodd(wbig.storage(), cfa::Layout{1, {b, s, h * d}, {s * h * d, h * d, 1}});
  const cfa::Tensor w = cfa::Tensor::from_host(in.w, {b, s, h * d}, g_stream);
  expect(bit_equal(a.node->bwd(a.input, a.out, w, g_stream).to_host(g_stream),
                   m.node->bwd(m.input, m.out, wodd, g_stream).to_host(g_stream)),
         "misaligned gradient: dqkv differs");
  // fused_attention with q at offset 1 and k transposed in (s, d) storage: both copied.
  const auto [q, k, v] = qkv_views(qkv, h, d);
  const auto [oq, ok, ov] = qkv_views(odd, h, d);
  expect(!cfa::float4_aligned(oq.layout()), "offset-1 view is not float4-aligned");
  const cfa::Tensor kt = k.contiguous(g_stream).transpose(2, 3).contiguous(g_stream).transpose(2, 3);
  expect(!cfa::float4_aligned(kt.layout()), "a d-strided view is not float4-aligned");
  const cfa::Applied f1 = cfa::fused_attention(q, k, v, 0.125f, false, g_stream);
  const cfa::Applied f2 = cfa::fused_attention(oq, kt, ov, 0.125f, false, g_stream);
  expect(f2.q.storage() != odd.storage() && f2.k.storage() != kt.storage(),
         "misaligned operands are copied");
  expect(bit_equal(f1.out.to_host(g_stream), f2.out.to_host(g_stream)),
         "fused_attention copy: outputs differ");
  const cfa::Tensor wr = w.reshape({b, s, h, d}, g_stream);
  const auto g1 = f1.node->bwd(f1.q, f1.k, f1.v, f1.raw, wr, g_stream);
  const auto g2 = f2.node->bwd(f2.q, f2.k, f2.v, f2.raw, wr, g_stream);
  for (int i = 0; i < 3; ++i) {
    expect(bit_equal(g1[i].to_host(g_stream), g2[i].to_host(g_stream)),
           "fused_attention copy: gradient " + std::to_string(i) + " differs");
  }
}

// The backward's gradients are views of one [b, s, 3, h, d] buffer, which is the projection's
// gradient (src/lib.rs:484-485): the two paths give the same dqkv bit for bit.
void gradient_views_share_the_qkv_layout() {
  const std::size_t b = 2, s = 40, h = 3, d = 64;
  const Inputs in = inputs(b, s, h, d);
  const cfa::Tensor qkv = cfa::Tensor::from_host(in.x, {b, s, 3 * h * d}, g_stream);
  const cfa::Tensor w = cfa::Tensor::from_host(in.w, {b, s, h * d}, g_stream);
  const auto [q, k, v] = qkv_views(qkv, h, d);
  const cfa::Applied f = cfa::fused_attention(q, k, v, 0.125f, false, g_stream);
  const auto g = f.node->bwd(f.q, f.k, f.v, f.raw, w.reshape({b, s, h, d}, g_stream), g_stream);
  for (int i = 0; i < 3; ++i) {
    expect(g[i].storage() == g[0].storage(), "one buffer");
    expect(g[i].layout().start_offset == i * h * d, "part offset");
    expect(g[i].stride() == Dims({s * 3 * h * d, d, 3 * h * d, 1}), "part strides");
  }
  const cfa::Tensor whole(g[0].storage(), cfa::Layout{0, {b, s, 3 * h * d}, {s * 3 * h * d, 3 * h * d, 1}});
  const cfa::QkvApplied a = cfa::fused_attention_qkv(qkv, h, 0.125f, false, g_stream);
  expect(bit_equal(whole.to_host(g_stream), a.node->bwd(a.input, a.out, w, g_stream).to_host(g_stream)),
         "the views' buffer differs from fused_attention_qkv's gradient");
}

// The strided gather behind contiguous(), to_host() and the copy fallbacks: every view of a
// [2, 3, 5, 7] tensor (transposes, a narrowed and squeezed slice, an offset) comes back in
// row-major order of its logical shape, as computed on the host.
void strided_copies_match_the_host() {
  const Dims shape{2, 3, 5, 7};
  std::vector<float> x(2 * 3 * 5 * 7);
  for (std::size_t i = 0; i < x.size(); ++i) x[i] = static_cast<float>(i);
  const cfa::Tensor t = cfa::Tensor::from_host(x, shape, g_stream);
  auto at = [&](std::size_t a, std::size_t b, std::size_t c, std::size_t d) {
    return x[((a * 3 + b) * 5 + c) * 7 + d];
  };
  // transpose(1, 3): [2, 7, 5, 3]
  std::vector<float> want;
  for (std::size_t a = 0; a < 2; ++a)
    for (std::size_t d = 0; d < 7; ++d)
      for (std::size_t c = 0; c < 5; ++c)
        for (std::size_t b = 0; b < 3; ++b) want.push_back(at(a, b, c, d));
  const cfa::Tensor tt = t.transpose(1, 3);
  expect(!tt.is_contiguous(), "a transposed view is strided");
  expect(tt.to_host(g_stream) == want, "transpose(1, 3) gathered wrong");
  // narrow(2, 1, 3).narrow(1, 2, 1).squeeze(1): [2, 3, 7] at an offset
  want.clear();
  for (std::size_t a = 0; a < 2; ++a)
    for (std::size_t c = 1; c < 4; ++c)
      for (std::size_t d = 0; d < 7; ++d) want.push_back(at(a, 2, c, d));
  const cfa::Tensor sl = t.narrow(2, 1, 3).narrow(1, 2, 1).squeeze(1);
  expect(sl.layout().start_offset == 2 * 35 + 7, "slice offset");
  const cfa::Tensor c = sl.contiguous(g_stream);
  expect(c.is_contiguous() && c.layout().start_offset == 0, "contiguous copy at offset 0");
  expect(c.to_host(g_stream) == want, "narrowed slice gathered wrong");
  // reshape of a strided view copies first; of a contiguous one it is a view
  const cfa::Tensor r = tt.reshape({2, 105}, g_stream);
  expect(r.storage() != t.storage(), "reshape of a strided view copies");
  expect(t.reshape({6, 35}, g_stream).storage() == t.storage(), "reshape of a contiguous view");
  want.clear();
  for (std::size_t a = 0; a < 2; ++a)
    for (std::size_t d = 0; d < 7; ++d)
      for (std::size_t cc = 0; cc < 5; ++cc)
        for (std::size_t b = 0; b < 3; ++b) want.push_back(at(a, b, cc, d));
  expect(r.to_host(g_stream) == want, "reshape copy order");
}

// Errors the C ABI raises (with the reference's messages) and the layer's own.
void gpu_errors() {
  const Inputs in = inputs(1, 8, 2, 48);
  const cfa::Tensor qkv48 = cfa::Tensor::from_host(in.x, {1, 8, 3 * 2 * 48}, g_stream);
  expect_error([&] { cfa::fused_attention_qkv(qkv48, 2, 0.1f, false, g_stream); }, "head_dim");
  const auto [q, k, v] = qkv_views(qkv48, 2, 48);
  expect_error([&] { cfa::fused_attention(q, k, v, 0.1f, false, g_stream); }, "head_dim");
  const Inputs ok = inputs(1, 8, 2, 64);
  const cfa::Tensor qkv = cfa::Tensor::from_host(ok.x, {1, 8, 3 * 2 * 64}, g_stream);
  expect_error([&] { cfa::fused_attention_qkv(qkv, 5, 0.1f, false, g_stream); },
               "fused_attention_qkv");
  const auto [q6, k6, v6] = qkv_views(qkv, 2, 64);
  const cfa::Tensor k_short = k6.narrow(2, 0, 7);
  expect_error([&] { cfa::fused_attention(q6, k_short, v6, 0.1f, false, g_stream); },
               "fused_attention");
  // O must be contiguous (src/lib.rs:347-351).
  const cfa::Applied f = cfa::fused_attention(q6, k6, v6, 0.1f, false, g_stream);
  const cfa::Tensor w = cfa::Tensor::from_host(std::vector<float>(8 * 2 * 64, 1.0f), {1, 8, 2, 64}, g_stream);
  expect_error([&] { f.node->bwd(q6, k6, v6, f.raw.transpose(1, 2), w, g_stream); },
               "O and L must be contiguous");
  expect_error([&] { f.node->bwd(q6, k6, v6, f.raw, w.reshape({1, 8, 128}, g_stream), g_stream); },
               "rank-4 gradient expected");
  const cfa::QkvApplied a = cfa::fused_attention_qkv(qkv, 2, 0.1f, false, g_stream);
  expect_error([&] { a.node->bwd(a.input, a.out, w, g_stream); }, "rank-3 gradient expected");
}

// --- CPU cases (no device call) ------------------------------------------------------------------

cfa::Tensor placeholder(const Dims& shape) {
  std::size_t n = 1;
  for (std::size_t x : shape) n *= x;
  Dims st(shape.size(), 1);
  for (std::size_t i = shape.size(); i-- > 1;) st[i - 1] = st[i] * shape[i];
  return cfa::Tensor(std::make_shared<cfa::Storage>(nullptr, n), cfa::Layout{0, shape, st});
}

// The views the ops build: qkv_views, the output's transposed view, the gradient parts.
void views_have_the_reference_layouts() {
  const std::size_t b = 2, s = 5, h = 3, d = 8;
  const cfa::Tensor qkv = placeholder({b, s, 3 * h * d});
  const auto [q, k, v] = qkv_views(qkv, h, d);
  expect(q.dims() == Dims({b, h, s, d}), "view dims");
  expect(k.layout().start_offset == h * d && v.layout().start_offset == 2 * h * d, "offsets");
  expect(q.stride() == Dims({s * 3 * h * d, d, 3 * h * d, 1}), "view strides");
  expect(cfa::float4_aligned(q.layout()) && cfa::float4_aligned(v.layout()), "views aligned");
  expect(!q.is_contiguous(), "views are strided");
  const cfa::Tensor raw = placeholder({b, s, h, d});
  expect(raw.transpose(1, 2).transpose(1, 2).is_contiguous(), "transpose twice");
  const cfa::Tensor dqkv = placeholder({b, s, 3, h, d});
  const cfa::Tensor dk = dqkv.narrow(2, 1, 1).squeeze(2).transpose(1, 2);
  expect(dk.dims() == Dims({b, h, s, d}) && dk.layout().start_offset == h * d &&
             dk.stride() == Dims({s * 3 * h * d, d, 3 * h * d, 1}),
         "gradient part layout");
  // Size-1 dims do not break contiguity.
  expect(placeholder({1, 4, 1, 8}).transpose(0, 2).is_contiguous(), "size-1 dims");
}

void alignment_predicates() {
  cfa::Layout l{0, {2, 3, 5, 64}, {960, 320, 64, 1}};
  expect(cfa::float4_aligned(l), "contiguous");
  l.start_offset = 2;
  expect(!cfa::float4_aligned(l), "offset 2");
  l.start_offset = 4;
  expect(cfa::float4_aligned(l), "offset 4");
  l.stride = {960, 320, 66, 1};
  expect(!cfa::float4_aligned(l), "seq stride 66");
  l.stride = {960, 320, 64, 2};
  expect(!cfa::float4_aligned(l), "d stride 2");
  expect(!cfa::float4_aligned(cfa::Layout{0, {2, 3, 64}, {192, 64, 1}}), "rank 3");
}

void errors_before_any_launch() {
  cfa::FusedAttention op(0.125f, false);
  const cfa::Tensor t = placeholder({1, 2, 8, 64});
  expect_error([&] { op.bwd(t, t, t, placeholder({1, 8, 2, 64}), placeholder({1, 8, 2, 64}), g_stream); },
               "fused_attention: backward before forward");
  expect_error([&] { op.saved_lse(); }, "fused_attention: backward before forward");
  cfa::FusedAttentionQkv qop(2, 0.125f, false);
  expect_error([&] { qop.bwd(placeholder({1, 8, 384}), placeholder({1, 8, 128}), placeholder({1, 8, 128}), g_stream); },
               "fused_attention: backward before forward");
  expect_error([&] { qop.fwd(placeholder({8, 384}), g_stream); },
               "fused_attention_qkv: a [b, s, 3 h d] tensor expected");
  expect_error([&] { op.fwd(placeholder({8, 64}), t, t, g_stream); },
               "fused_attention: a [b, h, s, d] tensor expected");
  expect_error([&] { placeholder({2, 3}).reshape({7}, g_stream); }, "cannot reshape");
  expect_error([&] { placeholder({2, 3}).narrow(1, 2, 2); }, "narrow out of range");
  expect_error([&] { placeholder({2, 3}).squeeze(0); }, "squeeze");
}

// Empty inputs are a no-op: nothing is allocated or launched (the C ABI returns at once).
void empty_inputs_are_a_no_op() {
  const cfa::Tensor qkv = cfa::Tensor::from_host({}, {0, 7, 3 * 2 * 64}, g_stream);
  const cfa::QkvApplied a = cfa::fused_attention_qkv(qkv, 2, 0.125f, false, g_stream);
  expect(a.out.dims() == Dims({0, 7, 128}), "empty output dims");
  expect(a.node->saved_lse().dims() == Dims({0, 2, 7}), "empty L dims");
  const cfa::Tensor q = cfa::Tensor::from_host({}, {1, 2, 0, 64}, g_stream);
  const cfa::Applied f = cfa::fused_attention(q, q, q, 0.125f, true, g_stream);
  expect(f.out.dims() == Dims({1, 2, 0, 64}), "empty fused_attention dims");
}

struct Case {
  const char* name;
  bool gpu;
  void (*fn)();
};

const Case kCases[] = {
    {"views_have_the_reference_layouts", false, views_have_the_reference_layouts},
    {"alignment_predicates", false, alignment_predicates},
    {"errors_before_any_launch", false, errors_before_any_launch},
    {"empty_inputs_are_a_no_op", false, empty_inputs_are_a_no_op},
    {"gpu_matches_oracle", true, gpu_matches_oracle},
    {"gpu_other_head_dims", true, gpu_other_head_dims},
    {"outputs_are_merge_heads_ready", true, outputs_are_merge_heads_ready},
    {"backward_twice_over_one_graph", true, backward_twice_over_one_graph},
    {"backward_is_deterministic", true, backward_is_deterministic},
    {"cached_blocks_are_reused_and_released", true, cached_blocks_are_reused_and_released},
    {"copy_fallbacks_match_aligned_operands", true, copy_fallbacks_match_aligned_operands},
    {"gradient_views_share_the_qkv_layout", true, gradient_views_share_the_qkv_layout},
    {"strided_copies_match_the_host", true, strided_copies_match_the_host},
    {"gpu_errors", true, gpu_errors},
};

}  // namespace

int main(int argc, char** argv) {
  bool gpu = false, cpu = false;
  std::string only;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    if (a == "--gpu") gpu = true;
    else if (a == "--cpu") cpu = true;
    else if (a == "--only" && i + 1 < argc) only = argv[++i];
    else {
      std::fprintf(stderr, "usage: %s --cpu | --gpu [--only NAME]\n", argv[0]);
      return 2;
    }
  }
  if (gpu == cpu) {
    std::fprintf(stderr, "usage: %s --cpu | --gpu [--only NAME]\n", argv[0]);
    return 2;
  }
  if (gpu && hipStreamCreate(&g_stream) != hipSuccess) {
    std::fprintf(stderr, "no HIP device\n");
    return 3;
  }
  int failed = 0, ran = 0;
  for (const Case& c : kCases) {
    if (c.gpu != gpu || (!only.empty() && only != c.name)) continue;
    std::printf("%s ...\n", c.name);
    std::fflush(stdout);
    ++ran;
    try {
      c.fn();
      std::printf("PASS %s\n", c.name);
    } catch (const Failure& f) {
      std::printf("FAIL %s: %s\n", c.name, f.what.c_str());
      ++failed;
    } catch (const std::exception& e) {
      std::printf("FAIL %s: exception: %s\n", c.name, e.what());
      ++failed;
    }
    std::fflush(stdout);
  }
  if (gpu) {
    (void)hipStreamSynchronize(g_stream);
    (void)hipStreamDestroy(g_stream);
  }
  std::printf("%d of %d passed\n", ran - failed, ran);
  return failed == 0 && ran > 0 ? 0 : 1;
}
