// candle_fused_attn.hpp -- the reference crate's op layer (src/lib.rs) in C++, over the C ABI of
// libfattn.so (include/fattn.h).
//
// The reference wraps its CUDA kernels in two candle custom ops: FusedAttentionQkv (CustomOp1,
// src/lib.rs:493-590) and FusedAttention (CustomOp3, src/lib.rs:382-491), reached through
// fused_attention_qkv (src/lib.rs:110-125) and fused_attention (src/lib.rs:143-161). Each op keeps
// the forward's row log-sum-exp L behind a mutex for its backward (src/lib.rs:301-315), copies an
// operand the kernels cannot read in place (src/lib.rs:110-118, :163-178, :368-380), and reports
// failures as errors prefixed `fused_attention:` / `fused_attention_qkv:`. This header is the same
// layer for C++ callers on MI355X: Tensor stands in for a candle Tensor (a device storage plus a
// Layout: start offset, shape, strides, all in f32 elements), the op objects for the nodes candle
// keeps in its autograd graph, and Error for candle_core::Error.
//
// Device memory of outputs, copies and the backward workspace is cached per stream (a caching
// allocator, as candle's and torch's are): a tensor's storage, when its last view goes, is kept
// for the next storage of the same size on the same stream, reused with no HIP call (stream order
// makes its earlier users finish first); a size not cached comes stream-ordered from a memory pool
// this layer keeps per device (hipMallocFromPoolAsync). So a steady-state step allocates nothing.
// The memory is held until the process ends or release_cached_blocks() gives it back; call that
// before destroying a stream this layer allocated on (its blocks are kept under the stream's
// handle, which a later stream may reuse). Each op node also keeps its backward workspace between
// backwards on one stream. Every launch is asynchronous on the caller's stream, so that stream must
// outlive the tensors allocated on it. There is no CPU path: the operators run on the HIP device
// only.
#ifndef CANDLE_FUSED_ATTN_HPP
#define CANDLE_FUSED_ATTN_HPP

#include <hip/hip_runtime.h>

#include <array>
#include <cstddef>
#include <memory>
#include <mutex>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

namespace candle_fused_attn {

// The head dimension the reference's kernels are specialised for (src/lib.rs:91); the kernels
// here also take 32 and 128.
constexpr std::size_t kCudaHeadDim = 64;

// A failure of an operator; the message carries the reference's prefix.
class Error : public std::runtime_error {
 public:
  explicit Error(const std::string& msg) : std::runtime_error(msg) {}
};

// Device memory for f32 values: owned (taken from and given back to the layer's cache for the
// stream it was taken on) or a caller's (never freed).
class Storage {
 public:
  Storage(std::size_t n, hipStream_t stream);  // n floats for use on `stream`
  Storage(float* external, std::size_t n);     // wraps memory the caller owns
  ~Storage();
  Storage(const Storage&) = delete;
  Storage& operator=(const Storage&) = delete;
  float* data() const { return p_; }
  std::size_t size() const { return n_; }

 private:
  float* p_ = nullptr;
  std::size_t n_ = 0;
  hipStream_t stream_ = nullptr;
  bool owned_ = false;
};

// Gives the cached device memory back to the layer's pool (stream-ordered, after the work already
// on each block's stream); returns the bytes given back. Tensors still alive keep theirs.
std::size_t release_cached_blocks();

// What a candle Layout holds.
struct Layout {
  std::size_t start_offset = 0;
  std::vector<std::size_t> shape, stride;
  std::size_t elem_count() const;
  bool is_contiguous() const;
};

// A strided f32 tensor on one HIP device (a view of a shared storage).
class Tensor {
 public:
  Tensor() = default;
  Tensor(std::shared_ptr<Storage> storage, Layout layout);
  // A new contiguous tensor (uninitialised).
  static Tensor empty(const std::vector<std::size_t>& shape, hipStream_t stream);
  // A contiguous copy of host values.
  static Tensor from_host(const std::vector<float>& values, const std::vector<std::size_t>& shape,
                          hipStream_t stream);

  const Layout& layout() const { return layout_; }
  const std::vector<std::size_t>& dims() const { return layout_.shape; }
  const std::vector<std::size_t>& stride() const { return layout_.stride; }
  std::size_t rank() const { return layout_.shape.size(); }
  bool is_contiguous() const { return layout_.is_contiguous(); }
  const std::shared_ptr<Storage>& storage() const { return storage_; }
  // The storage's base pointer (the layout's start offset is separate, as in candle).
  float* storage_ptr() const { return storage_ ? storage_->data() : nullptr; }

  // Views (no copy).
  Tensor narrow(std::size_t dim, std::size_t start, std::size_t len) const;
  Tensor transpose(std::size_t a, std::size_t b) const;
  Tensor squeeze(std::size_t dim) const;
  // A reshape of a contiguous tensor (a view); a non-contiguous one is copied first.
  Tensor reshape(const std::vector<std::size_t>& shape, hipStream_t stream) const;
  // `*this` if contiguous, else a contiguous copy (a strided gather on the device).
  Tensor contiguous(hipStream_t stream) const;
  // The values in logical (row-major) order; synchronises `stream`.
  std::vector<float> to_host(hipStream_t stream) const;

 private:
  std::shared_ptr<Storage> storage_;
  Layout layout_;
};

// Whether the kernels read a [b, h, s, d] layout in place: offset and (batch, head, seq) strides
// multiples of 4 floats, d contiguous (src/lib.rs:163-168).
bool float4_aligned(const Layout& l);

// The backward workspace an op node keeps between backwards. The reference allocates its
// temporaries per backward and drops them at return (src/cuda.rs:200-209); kept here, a
// steady-state backward takes none. A backward takes the kept workspace out while it enqueues its
// launches (a concurrent backward on the same node finds none and takes a new one, so no two
// backwards share a workspace) and gives it back after; a backward on another stream, or needing
// more bytes, takes a new one (the old one is freed stream-ordered on its own stream).
class WorkspaceCache {
 public:
  struct Lease {
    std::shared_ptr<Storage> ws;
    std::size_t bytes = 0;
    hipStream_t stream = nullptr;
  };
  // The workspace for a (b, h, s, d) backward on `stream` (fattn_bwd_workspace_bytes).
  Lease take(std::size_t b, std::size_t h, std::size_t s, std::size_t d, hipStream_t stream);
  // Keeps `lease` for the next backward (the larger one, if one was given back meanwhile).
  void give_back(Lease lease);

 private:
  std::mutex mu_;
  Lease kept_;
};

// The qkv-in, merged-out op (FusedAttentionQkv, src/lib.rs:493-590).
class FusedAttentionQkv {
 public:
  FusedAttentionQkv(std::size_t heads, float scale, bool causal)
      : heads_(heads), scale_(scale), causal_(causal) {}
  const char* name() const { return "fused-attention-qkv"; }
  // cuda_fwd: qkv [b, s, 3 h d] (rows float4-aligned, last stride 1) -> out [b, s, h d]; keeps L.
  Tensor fwd(const Tensor& qkv, hipStream_t stream);
  // bwd: the projection's gradient [b, s, 3 h d] from the forward's input and output and the
  // output's gradient (copied first if its rows are not float4-aligned).
  Tensor bwd(const Tensor& qkv, const Tensor& res, const Tensor& grad_res, hipStream_t stream);
  // The forward's L [b, h, s] (an error before the forward).
  Tensor saved_lse() const;

 private:
  std::size_t heads_;
  float scale_;
  bool causal_;
  mutable std::mutex mu_;
  std::optional<Tensor> lse_;
  WorkspaceCache ws_;
};

// The [b, h, s, d]-in, [b, s, h, d]-out op (FusedAttention, src/lib.rs:382-491).
class FusedAttention {
 public:
  FusedAttention(float scale, bool causal) : scale_(scale), causal_(causal) {}
  const char* name() const { return "fused-attention"; }
  // cuda_fwd: q, k, v [b, h, s, d], float4-aligned -> the raw output [b, s, h, d]; keeps L.
  Tensor fwd(const Tensor& q, const Tensor& k, const Tensor& v, hipStream_t stream);
  // bwd: dQ, dK, dV, each a [b, h, s, d] view of one [b, s, 3, h, d] buffer, from the gradient
  // of the raw [b, s, h, d] output.
  std::array<Tensor, 3> bwd(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& res,
                            const Tensor& grad_res, hipStream_t stream);
  Tensor saved_lse() const;

 private:
  float scale_;
  bool causal_;
  mutable std::mutex mu_;
  std::optional<Tensor> lse_;
  WorkspaceCache ws_;
};

// fused_attention_qkv (src/lib.rs:110-125): the output [b, s, h d] and the op node holding L
// (candle keeps it in the autograd graph; here the caller does, for `node->bwd`). `input` is the
// tensor the op read: qkv itself, or its contiguous copy when qkv's rows are not float4-aligned.
struct QkvApplied {
  Tensor out;
  std::shared_ptr<FusedAttentionQkv> node;
  Tensor input;
};
QkvApplied fused_attention_qkv(const Tensor& qkv, std::size_t heads, float scale, bool causal,
                               hipStream_t stream);

// fused_attention (src/lib.rs:143-161): the output [b, h, s, d] (a transposed view of a contiguous
// [b, s, h, d] buffer), its raw [b, s, h, d] form, the op node, and the operands it read.
struct Applied {
  Tensor out;
  Tensor raw;
  std::shared_ptr<FusedAttention> node;
  Tensor q, k, v;
};
Applied fused_attention(const Tensor& q, const Tensor& k, const Tensor& v, float scale,
                        bool causal, hipStream_t stream);

}  // namespace candle_fused_attn

#endif  // CANDLE_FUSED_ATTN_HPP
