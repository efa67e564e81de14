// candle_fused_attn.cpp -- the op layer of candle_fused_attn.hpp over libfattn.so's C ABI.
//
// The geometry, shape, head_dim and alignment checks are the C ABI's (they carry the reference's
// conditions and messages, src/lib.rs:181-220, :420-447, :526-550); this layer adds what
// src/lib.rs does around them: the copy fallbacks, the saved L and its errors, output and
// workspace allocation, and the gradient views.
#include "candle_fused_attn.hpp"

#include <algorithm>
#include <cstdint>
#include <functional>
#include <map>
#include <numeric>
#include <utility>

#include "fattn.h"

namespace candle_fused_attn {
namespace {

[[noreturn]] void fail(const std::string& msg) { throw Error(msg); }

void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) fail(std::string("fused_attention: ") + what + ": " + hipGetErrorString(e));
}

// A failed C-ABI call: its message (prefixed like the reference's) as the error.
void check_abi(int rc) {
  if (rc != 0) {
    const char* msg = fattn_last_error();
    fail(msg && *msg ? msg : "fused_attention: error " + std::to_string(rc));
  }
}

std::vector<std::size_t> row_major(const std::vector<std::size_t>& shape) {
  std::vector<std::size_t> st(shape.size(), 1);
  for (std::size_t i = shape.size(); i-- > 1;) st[i - 1] = st[i] * shape[i];
  return st;
}

std::string dims_str(const std::vector<std::size_t>& v) {
  std::string s = "[";
  for (std::size_t i = 0; i < v.size(); ++i) s += (i ? ", " : "") + std::to_string(v[i]);
  return s + "]";
}

std::vector<int64_t> i64(const std::vector<std::size_t>& v) {
  return std::vector<int64_t>(v.begin(), v.end());
}

// A strided gather into a contiguous buffer: dst[i] = src[offset(i)], i in row-major order.
constexpr int kMaxRank = 8;
struct GatherArgs {
  const float* src;
  float* dst;
  int64_t n;
  int rank;
  int64_t shape[kMaxRank];
  int64_t stride[kMaxRank];
};

__global__ void gather_kernel(GatherArgs a) {
  const int64_t step = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < a.n;
       i += step) {
    int64_t rem = i, off = 0;
    for (int d = a.rank - 1; d >= 0; --d) {
      off += (rem % a.shape[d]) * a.stride[d];
      rem /= a.shape[d];
    }
    a.dst[i] = a.src[off];
  }
}

// The largest element offset a layout reaches (its start for an empty one).
std::size_t last_offset(const Layout& l) {
  std::size_t off = l.start_offset;
  for (std::size_t i = 0; i < l.shape.size(); ++i) {
    if (l.shape[i] == 0) return l.start_offset;
    off += (l.shape[i] - 1) * l.stride[i];
  }
  return off;
}

// Every element a layout reaches lies in its storage (candle's layouts do by construction; a
// Tensor built here from a raw Layout is checked before a kernel reads it).
void check_fits(const Tensor& t) {
  const Layout& l = t.layout();
  if (l.elem_count() == 0) return;
  if (!t.storage() || last_offset(l) >= t.storage()->size()) {
    fail("fused_attention: layout outside its storage");
  }
}

// A fresh contiguous copy at offset 0 (what the reference's copy fallbacks need: candle's
// contiguous() keeps a contiguous tensor at a misaligned offset as it is).
Tensor fresh_copy(const Tensor& t, hipStream_t stream) {
  const Layout& l = t.layout();
  Tensor out = Tensor::empty(l.shape, stream);
  const std::size_t n = l.elem_count();
  if (n == 0) return out;
  check_fits(t);
  if (l.shape.size() > static_cast<std::size_t>(kMaxRank)) fail("fused_attention: rank above 8");
  GatherArgs a{};
  a.src = t.storage_ptr() + l.start_offset;
  a.dst = out.storage_ptr();
  a.n = static_cast<int64_t>(n);
  a.rank = static_cast<int>(l.shape.size());
  for (int d = 0; d < a.rank; ++d) {
    a.shape[d] = static_cast<int64_t>(l.shape[d]);
    a.stride[d] = static_cast<int64_t>(l.stride[d]);
  }
  const int64_t blocks = std::min<int64_t>((a.n + 255) / 256, 4096);
  hipLaunchKernelGGL(gather_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
  check_hip(hipGetLastError(), "copy launch");
  return out;
}

// src/lib.rs:370-380: the gradient itself when its offset is a multiple of 4, its last stride 1
// and every other stride 1 or a multiple of 4; else a copy.
Tensor aligned_grad(const Tensor& g, hipStream_t stream) {
  const Layout& l = g.layout();
  bool ok = l.start_offset % 4 == 0 && (l.stride.empty() || l.stride.back() == 1);
  for (std::size_t s : l.stride) ok = ok && (s == 1 || s % 4 == 0);
  return ok ? g : fresh_copy(g, stream);
}

// save / saved (src/lib.rs:301-315): L is kept for the backward and read, not consumed.
void save(std::mutex& mu, std::optional<Tensor>& slot, const Tensor& l) {
  std::lock_guard<std::mutex> lock(mu);
  slot = l;
}

Tensor saved(std::mutex& mu, const std::optional<Tensor>& slot) {
  std::lock_guard<std::mutex> lock(mu);
  if (!slot) fail("fused_attention: backward before forward");
  return *slot;
}

// The layer's memory pool on the device that runs `stream` (the null stream: the current
// device), made on first use: a stream-ordered pool whose release threshold is the maximum, so
// memory given back stays in the pool for later allocations.
hipMemPool_t device_pool(hipStream_t stream) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static hipMemPool_t pools[kMaxDevices] = {};
  int dev = 0;
  check_hip(stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev), "device of stream");
  if (dev < 0 || dev >= kMaxDevices) fail("fused_attention: device index out of range");
  std::lock_guard<std::mutex> lock(mu);
  if (pools[dev] == nullptr) {
    hipMemPoolProps props{};
    props.allocType = hipMemAllocationTypePinned;
    props.handleTypes = hipMemHandleTypeNone;
    props.location.type = hipMemLocationTypeDevice;
    props.location.id = dev;
    hipMemPool_t pool = nullptr;
    check_hip(hipMemPoolCreate(&pool, &props), "memory pool");
    uint64_t keep = UINT64_MAX;
    check_hip(hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep),
              "memory pool threshold");
    pools[dev] = pool;
  }
  return pools[dev];
}

}  // namespace

// --- the kept backward workspace -----------------------------------------------------------------

WorkspaceCache::Lease WorkspaceCache::take(std::size_t b, std::size_t h, std::size_t s,
                                           std::size_t d, hipStream_t stream) {
  const std::size_t bytes = fattn_bwd_workspace_bytes(
      static_cast<int64_t>(b), static_cast<int64_t>(h), static_cast<int64_t>(s),
      static_cast<int64_t>(d));
  Lease kept;
  {
    std::lock_guard<std::mutex> lock(mu_);
    std::swap(kept, kept_);
  }
  if (kept.ws && kept.stream == stream && kept.bytes >= bytes) {
    kept.bytes = bytes;  // the size this backward asks for (its chunks follow from it)
    return kept;
  }
  Lease fresh;
  fresh.ws = std::make_shared<Storage>(std::max<std::size_t>(bytes, 256) / sizeof(float) + 1,
                                       stream);
  fresh.bytes = bytes;
  fresh.stream = stream;
  return fresh;
}

void WorkspaceCache::give_back(Lease lease) {
  if (!lease.ws) return;
  lease.bytes = lease.ws->size() * sizeof(float);
  std::lock_guard<std::mutex> lock(mu_);
  if (!kept_.ws || kept_.bytes < lease.bytes) std::swap(kept_, lease);
}

// --- Storage, Layout, Tensor -------------------------------------------------------------------

// --- device memory: a block cache over the layer's pool --------------------------------------------

namespace {

// Blocks given back by Storage, kept per (stream, size) for the next Storage of that size on that
// stream: taken and given back with no HIP call and no work on the stream (stream order makes a
// block's earlier users finish before its next user starts). Only a block of a size not cached
// comes from the pool (stream-ordered). The stream-ordered calls cost the host about 35 us each,
// so that at b 64 h 6 s 240 a step's three allocations and frees made the host, not the GPU, set
// the step's time (0.208 ms per step, the GPU's work 0.190 ms); cached, the host enqueues a step
// in 0.010 ms.
std::mutex g_cache_mu;
std::map<std::pair<hipStream_t, std::size_t>, std::vector<float*>> g_cache;

float* take_block(std::size_t n, hipStream_t stream) {
  {
    std::lock_guard<std::mutex> lock(g_cache_mu);
    auto it = g_cache.find({stream, n});
    if (it != g_cache.end() && !it->second.empty()) {
      float* p = it->second.back();
      it->second.pop_back();
      return p;
    }
  }
  void* p = nullptr;
  check_hip(hipMallocFromPoolAsync(&p, n * sizeof(float), device_pool(stream), stream),
            "allocation");
  return static_cast<float*>(p);
}

void give_block(float* p, std::size_t n, hipStream_t stream) {
  std::lock_guard<std::mutex> lock(g_cache_mu);
  g_cache[{stream, n}].push_back(p);
}

}  // namespace

std::size_t release_cached_blocks() {
  std::map<std::pair<hipStream_t, std::size_t>, std::vector<float*>> blocks;
  {
    std::lock_guard<std::mutex> lock(g_cache_mu);
    blocks.swap(g_cache);
  }
  std::size_t n = 0;
  for (auto& [key, ps] : blocks) {
    for (float* p : ps) {
      // Given back to the pool after the work already on the block's stream.
      check_hip(hipFreeAsync(p, key.first), "release");
      n += key.second * sizeof(float);
    }
  }
  return n;
}

Storage::Storage(std::size_t n, hipStream_t stream) : n_(n), stream_(stream), owned_(true) {
  if (n > 0) p_ = take_block(n, stream);
}

Storage::Storage(float* external, std::size_t n) : p_(external), n_(n), owned_(false) {}

Storage::~Storage() {
  if (owned_ && p_) give_block(p_, n_, stream_);
}

std::size_t Layout::elem_count() const {
  return std::accumulate(shape.begin(), shape.end(), std::size_t{1}, std::multiplies<>());
}

bool Layout::is_contiguous() const {
  std::size_t expect = 1;
  for (std::size_t i = shape.size(); i-- > 0;) {
    if (shape[i] != 1 && stride[i] != expect) return false;
    expect *= shape[i];
  }
  return true;
}

Tensor::Tensor(std::shared_ptr<Storage> storage, Layout layout)
    : storage_(std::move(storage)), layout_(std::move(layout)) {
  if (layout_.stride.size() != layout_.shape.size()) fail("fused_attention: shape/stride rank");
}

Tensor Tensor::empty(const std::vector<std::size_t>& shape, hipStream_t stream) {
  Layout l{0, shape, row_major(shape)};
  return Tensor(std::make_shared<Storage>(l.elem_count(), stream), l);
}

Tensor Tensor::from_host(const std::vector<float>& values, const std::vector<std::size_t>& shape,
                         hipStream_t stream) {
  Tensor t = empty(shape, stream);
  if (values.size() != t.layout().elem_count()) fail("fused_attention: host data/shape mismatch");
  if (!values.empty()) {
    check_hip(hipMemcpyAsync(t.storage_ptr(), values.data(), values.size() * sizeof(float),
                             hipMemcpyHostToDevice, stream),
              "host copy");
    check_hip(hipStreamSynchronize(stream), "host copy");
  }
  return t;
}

Tensor Tensor::narrow(std::size_t dim, std::size_t start, std::size_t len) const {
  if (dim >= rank() || start + len > layout_.shape[dim]) fail("fused_attention: narrow out of range");
  Layout l = layout_;
  l.start_offset += start * l.stride[dim];
  l.shape[dim] = len;
  return Tensor(storage_, l);
}

Tensor Tensor::transpose(std::size_t a, std::size_t b) const {
  if (a >= rank() || b >= rank()) fail("fused_attention: transpose out of range");
  Layout l = layout_;
  std::swap(l.shape[a], l.shape[b]);
  std::swap(l.stride[a], l.stride[b]);
  return Tensor(storage_, l);
}

Tensor Tensor::squeeze(std::size_t dim) const {
  if (dim >= rank() || layout_.shape[dim] != 1) fail("fused_attention: squeeze of a dim not 1");
  Layout l = layout_;
  l.shape.erase(l.shape.begin() + static_cast<std::ptrdiff_t>(dim));
  l.stride.erase(l.stride.begin() + static_cast<std::ptrdiff_t>(dim));
  return Tensor(storage_, l);
}

Tensor Tensor::reshape(const std::vector<std::size_t>& shape, hipStream_t stream) const {
  Layout l{0, shape, row_major(shape)};
  if (l.elem_count() != layout_.elem_count()) {
    fail("fused_attention: cannot reshape " + dims_str(layout_.shape) + " to " + dims_str(shape));
  }
  const Tensor src = is_contiguous() ? *this : fresh_copy(*this, stream);
  l.start_offset = src.layout_.start_offset;
  return Tensor(src.storage_, l);
}

Tensor Tensor::contiguous(hipStream_t stream) const {
  return is_contiguous() ? *this : fresh_copy(*this, stream);
}

std::vector<float> Tensor::to_host(hipStream_t stream) const {
  const Tensor c = contiguous(stream);
  std::vector<float> out(layout_.elem_count());
  if (!out.empty()) {
    check_hip(hipMemcpyAsync(out.data(), c.storage_ptr() + c.layout_.start_offset,
                             out.size() * sizeof(float), hipMemcpyDeviceToHost, stream),
              "device copy");
  }
  check_hip(hipStreamSynchronize(stream), "device copy");
  return out;
}

bool float4_aligned(const Layout& l) {
  return l.shape.size() == 4 && l.start_offset % 4 == 0 && l.stride[3] == 1 &&
         l.stride[0] % 4 == 0 && l.stride[1] % 4 == 0 && l.stride[2] % 4 == 0;
}

// --- the ops -------------------------------------------------------------------------------------

Tensor FusedAttentionQkv::fwd(const Tensor& qkv, hipStream_t stream) {
  const Layout& l = qkv.layout();
  if (l.shape.size() != 3) {
    fail("fused_attention_qkv: a [b, s, 3 h d] tensor expected, got shape " + dims_str(l.shape));
  }
  check_fits(qkv);
  const std::size_t b = l.shape[0], s = l.shape[1], hd = l.shape[2] / 3;
  Tensor out = Tensor::empty({b, s, hd}, stream);
  Tensor lse = Tensor::empty({b, heads_, s}, stream);
  const auto shape = i64(l.shape), strides = i64(l.stride);
  check_abi(fattn_qkv_forward(qkv.storage_ptr(), static_cast<int64_t>(l.start_offset),
                              shape.data(), strides.data(), static_cast<int64_t>(heads_), scale_,
                              causal_ ? 1 : 0, out.storage_ptr(), lse.storage_ptr(), stream));
  save(mu_, lse_, lse);
  return out;
}

Tensor FusedAttentionQkv::bwd(const Tensor& qkv, const Tensor& res, const Tensor& grad_res,
                              hipStream_t stream) {
  const Tensor l = saved(mu_, lse_);
  const Tensor grad = aligned_grad(grad_res, stream);
  const Layout& ql = qkv.layout();
  if (ql.shape.size() != 3) {
    fail("fused_attention_qkv: a [b, s, 3 h d] tensor expected, got shape " + dims_str(ql.shape));
  }
  if (grad.rank() != 3) fail("fused_attention_qkv: rank-3 gradient expected");
  if (!res.is_contiguous() || !l.is_contiguous()) {
    fail("fused_attention: O and L must be contiguous");
  }
  for (const Tensor* t : {&qkv, &res, &grad}) check_fits(*t);
  const std::size_t b = ql.shape[0], s = ql.shape[1], three_hd = ql.shape[2];
  const std::size_t d = heads_ ? three_hd / 3 / heads_ : 0;
  // The forward's output and L of this projection (the kernels read O and L whole).
  if (res.layout().elem_count() != b * s * heads_ * d || l.layout().elem_count() != b * heads_ * s) {
    fail("fused_attention_qkv: O and L do not match the projection's shape");
  }
  Tensor dqkv = Tensor::empty({b, s, three_hd}, stream);
  WorkspaceCache::Lease ws = ws_.take(b, heads_, s, d, stream);
  const auto shape = i64(ql.shape), strides = i64(ql.stride);
  const auto gshape = i64(grad.dims()), gstrides = i64(grad.stride());
  check_abi(fattn_qkv_backward(
      qkv.storage_ptr(), static_cast<int64_t>(ql.start_offset), shape.data(), strides.data(),
      static_cast<int64_t>(heads_), scale_, causal_ ? 1 : 0,
      res.storage_ptr() + res.layout().start_offset, l.storage_ptr() + l.layout().start_offset,
      grad.storage_ptr(), static_cast<int64_t>(grad.layout().start_offset), gshape.data(),
      gstrides.data(), dqkv.storage_ptr(), ws.ws->data(), ws.bytes, stream));
  ws_.give_back(std::move(ws));
  return dqkv;
}

Tensor FusedAttentionQkv::saved_lse() const { return saved(mu_, lse_); }

Tensor FusedAttention::fwd(const Tensor& q, const Tensor& k, const Tensor& v, hipStream_t stream) {
  for (const Tensor* t : {&q, &k, &v}) {
    if (t->rank() != 4) {
      fail("fused_attention: a [b, h, s, d] tensor expected, got shape " + dims_str(t->dims()));
    }
  }
  for (const Tensor* t : {&q, &k, &v}) check_fits(*t);
  const auto& dims = q.dims();
  const std::size_t b = dims[0], h = dims[1], s = dims[2], d = dims[3];
  Tensor raw = Tensor::empty({b, s, h, d}, stream);
  Tensor lse = Tensor::empty({b, h, s}, stream);
  std::vector<int64_t> sh[3], st[3];
  const Tensor* ops[3] = {&q, &k, &v};
  for (int i = 0; i < 3; ++i) {
    sh[i] = i64(ops[i]->dims());
    st[i] = i64(ops[i]->stride());
  }
  check_abi(fattn_forward(q.storage_ptr(), static_cast<int64_t>(q.layout().start_offset),
                          sh[0].data(), st[0].data(), k.storage_ptr(),
                          static_cast<int64_t>(k.layout().start_offset), sh[1].data(),
                          st[1].data(), v.storage_ptr(),
                          static_cast<int64_t>(v.layout().start_offset), sh[2].data(),
                          st[2].data(), scale_, causal_ ? 1 : 0, raw.storage_ptr(),
                          lse.storage_ptr(), stream));
  save(mu_, lse_, lse);
  return raw;
}

std::array<Tensor, 3> FusedAttention::bwd(const Tensor& q, const Tensor& k, const Tensor& v,
                                          const Tensor& res, const Tensor& grad_res,
                                          hipStream_t stream) {
  const Tensor l = saved(mu_, lse_);
  const Tensor grad = aligned_grad(grad_res, stream);
  if (q.rank() != 4) {
    fail("fused_attention: a [b, h, s, d] tensor expected, got shape " + dims_str(q.dims()));
  }
  if (grad.rank() != 4) fail("fused_attention: rank-4 gradient expected");
  if (!res.is_contiguous() || !l.is_contiguous()) {
    fail("fused_attention: O and L must be contiguous");
  }
  for (const Tensor* t : {&q, &k, &v, &res, &grad}) check_fits(*t);
  const auto& dims = q.dims();
  const std::size_t b = dims[0], h = dims[1], s = dims[2], d = dims[3];
  if (res.layout().elem_count() != b * s * h * d || l.layout().elem_count() != b * h * s) {
    fail("fused_attention: O and L do not match q's shape");
  }
  Tensor dqkv = Tensor::empty({b, s, 3, h, d}, stream);
  WorkspaceCache::Lease ws = ws_.take(b, h, s, d, stream);
  std::vector<int64_t> sh[3], st[3];
  const Tensor* ops[3] = {&q, &k, &v};
  for (int i = 0; i < 3; ++i) {
    sh[i] = i64(ops[i]->dims());
    st[i] = i64(ops[i]->stride());
  }
  const auto gshape = i64(grad.dims()), gstrides = i64(grad.stride());
  check_abi(fattn_backward(
      q.storage_ptr(), static_cast<int64_t>(q.layout().start_offset), sh[0].data(), st[0].data(),
      k.storage_ptr(), static_cast<int64_t>(k.layout().start_offset), sh[1].data(), st[1].data(),
      v.storage_ptr(), static_cast<int64_t>(v.layout().start_offset), sh[2].data(), st[2].data(),
      scale_, causal_ ? 1 : 0, res.storage_ptr() + res.layout().start_offset,
      l.storage_ptr() + l.layout().start_offset, grad.storage_ptr(),
      static_cast<int64_t>(grad.layout().start_offset), gshape.data(), gstrides.data(),
      dqkv.storage_ptr(), ws.ws->data(), ws.bytes, stream));
  ws_.give_back(std::move(ws));
  // dQ, dK, dV: narrow views of the one buffer, each [b, h, s, d] (src/lib.rs:484-485).
  auto part = [&](std::size_t i) { return dqkv.narrow(2, i, 1).squeeze(2).transpose(1, 2); };
  return {part(0), part(1), part(2)};
}

Tensor FusedAttention::saved_lse() const { return saved(mu_, lse_); }

// --- the public functions ------------------------------------------------------------------------

QkvApplied fused_attention_qkv(const Tensor& qkv, std::size_t heads, float scale, bool causal,
                               hipStream_t stream) {
  // src/lib.rs:111-118: read in place when offset and [sb, ss] are multiples of 4 and the last
  // stride is 1; else a copy.
  const Layout& l = qkv.layout();
  const bool aligned = l.shape.size() != 3 ||
                       (l.start_offset % 4 == 0 && l.stride[2] == 1 && l.stride[0] % 4 == 0 &&
                        l.stride[1] % 4 == 0);
  QkvApplied r;
  r.input = aligned ? qkv : fresh_copy(qkv, stream);
  r.node = std::make_shared<FusedAttentionQkv>(heads, scale, causal);
  r.out = r.node->fwd(r.input, stream);
  return r;
}

Applied fused_attention(const Tensor& q, const Tensor& k, const Tensor& v, float scale,
                        bool causal, hipStream_t stream) {
  // float4_rows (src/lib.rs:170-178): each operand itself when float4-aligned, else a copy.
  auto rows = [&](const Tensor& t) {
    return t.rank() != 4 || float4_aligned(t.layout()) ? t : fresh_copy(t, stream);
  };
  Applied r;
  r.q = rows(q);
  r.k = rows(k);
  r.v = rows(v);
  r.node = std::make_shared<FusedAttention>(scale, causal);
  r.raw = r.node->fwd(r.q, r.k, r.v, stream);
  r.out = r.raw.transpose(1, 2);
  return r;
}

}  // namespace candle_fused_attn
