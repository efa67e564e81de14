// The C ABI (include/fattn.h): argument validation with the reference's conditions and
// messages, operand views, workspace layout, and the launches (fattn_kernels.hip).
//
// Validation runs before any HIP call, so a rejected call touches no device and needs none.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <numeric>
#include <atomic>
#include <chrono>
#include <cstdint>
#include <climits>
#include <random>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "fattn.h"
#include "fattn_internal.h"

namespace fattn {

Workspace workspace_layout(int64_t b, int64_t h, int64_t s, int64_t d) {
  auto up = [](size_t x) { return (x + 255) & ~static_cast<size_t>(255); };
  Workspace w{};
  const size_t rows = static_cast<size_t>(b * h * s);
  const size_t tiles = static_cast<size_t>(b * h * ((s + kBwdQueryTile - 1) / kBwdQueryTile));
  const size_t nkb = static_cast<size_t>((s + kBwdKeys - 1) / kBwdKeys);
  // The control words (ticket, guard word) first: their place is the same for every shape, so
  // fattn_bwd_status finds the guard word whichever way the workspace was used.
  w.ctrl_off = 0;
  w.d_off = up(64 * sizeof(int));
  w.turn_off = w.d_off + up(rows * sizeof(float));
  w.part_off = w.turn_off + up(tiles * sizeof(int));
  w.bytes_min = w.part_off;
  w.arrive_off = w.part_off + up(nkb * tiles * kBwdQueryTile * static_cast<size_t>(d) *
                                 sizeof(float));
  w.done_off = w.arrive_off + up(static_cast<size_t>(b * h) * nkb * sizeof(unsigned long long));
  w.epoch_off = w.done_off + up(tiles * sizeof(unsigned long long));
  w.bytes_split = w.epoch_off + 256;
  return w;
}

// The split step 2's workgroup slots on gfx950 (256 CUs): 3 per CU, 2 with 128-key blocks at
// d 64.
int64_t split_slots(int keys, int64_t d) {
  return (keys > kBwdKeys && d > 32 ? 2 : 3) * int64_t{256};
}

// The (b, h) pairs per chunk of the split dQ sum that a workspace of ws_bytes holds: b h when it
// holds the whole split; else, at d <= 64, from the most pairs whose split partials, arrival
// slots and done flags fit:
//   causal: equal chunks (the key blocks' own sums read the partials at device scope, so the
//     XCDs a chunk's key blocks run on do not matter);
//   non-causal: the most pairs whose key blocks fill whole rounds of the chip's workgroup slots
//     (every key block walks all query tiles, so a partial round idles slots; the last chunk
//     takes the rest);
// 0 when that is fewer than min_pairs. Steps 2 and 3 then run per chunk, each chunk's state at
// the start of the workspace (workspace_layout(1, chunk, s, d)).
int64_t split_chunk(int64_t b, int64_t h, int64_t s, int64_t d, size_t ws_bytes,
                    int64_t min_pairs, bool causal) {
  const int64_t total = b * h;
  if (workspace_layout(b, h, s, d).bytes_split <= ws_bytes) return total;
  if (d > 64) return 0;
  int64_t lo = 0, hi = total - 1;  // the split size grows with the pair count
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) / 2;
    if (workspace_layout(1, mid, s, d).bytes_split <= ws_bytes) {
      lo = mid;
    } else {
      hi = mid - 1;
    }
  }
  if (!causal) {
    const int keys = bwd_split_keys(b, h, s, static_cast<int>(d), 0);
    const int64_t nkb = (s + keys - 1) / keys, slots = split_slots(keys, d);
    const int64_t quantum = slots / std::gcd(slots, nkb);
    if (lo >= quantum) lo -= lo % quantum;
    return lo == 0 || lo < min_pairs ? 0 : lo;
  }
  if (lo == 0 || lo < min_pairs) return 0;
  // Equal chunks: ceil(total / chunks) <= lo.
  const int64_t chunks = (total + lo - 1) / lo;
  return (total + chunks - 1) / chunks;
}

// The fewest (b, h) pairs a chunk should hold. A chunk is one launch of step 2: with too few key
// blocks it runs at a fraction of the chip, so chunks of fewer pairs than this lose to the turn
// hand-over over all pairs (measured: b 4 h 16 s 8192 causal, chunks of 8 pairs 15.1 ms against
// 13.8 with turns). Non-causal: the chunk's key blocks fill the chip's workgroup slots at least
// once. Causal: the key blocks' walks shrink with the block index, so the slots' average work must
// be at least twice the longest walk (block 0's, all query tiles): four times the slots in key
// blocks.
int64_t min_chunk_pairs(int64_t b, int64_t h, int64_t s, int64_t d, bool causal) {
  const int keys = bwd_split_keys(b, h, s, static_cast<int>(d), causal ? 1 : 0);
  const int64_t nkb = (s + keys - 1) / keys;
  const int64_t blocks = (causal ? 4 : 1) * split_slots(keys, d);
  return (blocks + nkb - 1) / nkb;
}

// The workspace the library asks for within `limit` bytes: the whole split, else the split of the
// larger of the chunks each mask's rule takes (the size takes no mask; a run applies its own rule
// to the workspace it is given, and each rule's chunk fits in the larger one), else the turn
// hand-over's minimum (possibly over the limit: the caller decides).
size_t workspace_within(int64_t b, int64_t h, int64_t s, int64_t d, size_t limit) {
  const Workspace l = workspace_layout(b, h, s, d);
  if (l.bytes_split <= limit) return l.bytes_split;
  const int64_t c = std::max(
      split_chunk(b, h, s, d, limit, min_chunk_pairs(b, h, s, d, false), false),
      split_chunk(b, h, s, d, limit, min_chunk_pairs(b, h, s, d, true), true));
  return c > 0 ? workspace_layout(1, c, s, d).bytes_split : l.bytes_min;
}

}  // namespace fattn

namespace {

using fattn::View;

thread_local std::string g_error;

// A 64-bit value unique to each step 2 launch of this process (low 3 bits zero, for the XCD), the
// sequence starting at a random point: step 2's dQ sums tag their workspace state with it.
unsigned long long next_epoch() {
  static std::atomic<unsigned long long> counter{[] {
    std::random_device rd;
    return (static_cast<unsigned long long>(rd()) << 32) ^ rd() ^
           static_cast<unsigned long long>(
               std::chrono::steady_clock::now().time_since_epoch().count());
  }()};
  unsigned long long e = 0;
  while (e == 0) e = counter.fetch_add(1, std::memory_order_relaxed) << 3;
  return e;
}

int fail(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

// Whether the test hooks may act in this process: FATTN_TEST_HOOKS=1 in the environment when the
// library was loaded (read once, by the library's static initialisation).
const bool g_test_hooks = [] {
  const char* v = std::getenv("FATTN_TEST_HOOKS");
  return v != nullptr && std::strcmp(v, "1") == 0;
}();

int hooks_refused(const char* name) {
  return fail(FATTN_EINVAL, std::string("fused_attention: ") + name +
                                " is a test hook; it acts only when FATTN_TEST_HOOKS=1 was set "
                                "before the library loaded");
}

int ok() {
  g_error.clear();
  return 0;
}

int hip_fail(int err, const char* what) {
  g_error = std::string("fused_attention: ") + what + ": " +
            hipGetErrorString(static_cast<hipError_t>(err));
  return err;
}

std::string dims_str(const int64_t* x, int n) {
  std::string out = "[";
  for (int i = 0; i < n; ++i) {
    if (i) out += ", ";
    out += std::to_string(x[i]);
  }
  return out + "]";
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Kernel index range: every (b, h, s) index product and the grid stay inside int32, and the
// launch inside 2^32 threads.
int check_range(const char* who, int64_t b, int64_t h, int64_t s, int64_t d) {
  const int64_t lim = INT32_MAX;
  if (b > lim || h > lim || s > lim || b * h > lim || b * h * s > lim) {
    return fail(FATTN_ERANGE, std::string(who) + ": " + std::to_string(b) + " x " +
                                  std::to_string(h) + " x " + std::to_string(s) +
                                  " exceeds i32 indexing");
  }
  const int64_t grid_lim = (int64_t{1} << 32) / 256 - 1;
  const int dd = static_cast<int>(d);
  if (fattn::forward_blocks(b, h, s, 1, dd) > grid_lim ||
      fattn::forward_blocks(b, h, s, 0, dd) > grid_lim ||
      fattn::bwd_main_blocks(b, h, s) + fattn::bwd_dq_blocks(b, h, s) + 8 > grid_lim ||
      fattn::bwd_prep_blocks(b, h, s, dd) > grid_lim) {
    return fail(FATTN_ERANGE, std::string(who) + ": the grid for " + std::to_string(b) +
                                  " x " + std::to_string(h) + " x " + std::to_string(s) +
                                  " exceeds the launch limit");
  }
  return 0;
}

// The op level and the generic kernel-level entries: the head_dims the kernels are built for.
int check_head_dim(int64_t d) {
  if (!fattn::head_dim_supported(d)) {
    return fail(FATTN_EHEADDIM,
                "fused_attention: the HIP kernels take head_dim 32, 64 or 128, got " +
                    std::to_string(d));
  }
  return 0;
}

// The entries named after the reference's d64 kernels take exactly its head_dim
// (src/cuda.rs:85-93).
int check_head_dim64(int64_t d) {
  if (d != fattn::kHeadDim) {
    return fail(FATTN_EHEADDIM, "fused_attention: the HIP kernels take head_dim 64, got " +
                                    std::to_string(d));
  }
  return 0;
}

bool view_aligned(const View& v) {
  return aligned16(v.p) && v.sb % 4 == 0 && v.sh % 4 == 0 && v.ss % 4 == 0;
}

View make_view(const float* base, const int64_t st[3]) { return View{base, st[0], st[1], st[2]}; }

// The kernels address a (b, h) slice of an operand (and a batch of dqkv) with 32-bit byte or
// element offsets from a per-slice base.
bool slice_fits(const View& v, int64_t s, int64_t d) {
  return (s - 1) * v.ss * 4 + 4 * d <= int64_t{UINT32_MAX};
}

int slice_error(const char* who, int64_t s) {
  return fail(FATTN_ERANGE, std::string(who) + ": a (batch, head) slice of " + std::to_string(s) +
                                " rows spans more than 4 GiB");
}

// Shared body of the kernel-level forward.
int run_forward(const char* who, View q, View k, View v, float* o, float* lse, int64_t b,
                int64_t h, int64_t s, int64_t d, float scale, int causal, void* stream) {
  if (int rc = check_range(who, b, h, s, d)) return rc;
  if (!q.p || !k.p || !v.p || !o || !lse) {
    return fail(FATTN_EINVAL, std::string(who) + ": null operand");
  }
  if (!view_aligned(q) || !view_aligned(k) || !view_aligned(v) || !aligned16(o)) {
    return fail(FATTN_EALIGN, std::string(who) + ": rows must be 16-byte aligned");
  }
  if (!slice_fits(k, s, d) || !slice_fits(v, s, d)) return slice_error(who, s);
  const int err = fattn::launch_forward(q, k, v, o, lse, static_cast<int>(b),
                                        static_cast<int>(h), static_cast<int>(s),
                                        static_cast<int>(d), scale, causal ? 1 : 0, stream);
  if (err) return hip_fail(err, "forward launch");
  return ok();
}

struct WsParts {
  float* dsum;
  float* part;  // null: the workspace is too small for the split partials (turn hand-over)
  unsigned long long* arrive;  // split: step 2's dQ sums
  unsigned long long* done;
  unsigned long long* epoch;
  int* turn;
  int* ctrl;
};

int workspace_parts(const char* who, void* ws, size_t ws_bytes, int64_t b, int64_t h, int64_t s,
                    int64_t d, WsParts* out) {
  const fattn::Workspace l = fattn::workspace_layout(b, h, s, d);
  if (!ws || (reinterpret_cast<uintptr_t>(ws) & 255u) != 0 || ws_bytes < l.bytes_min) {
    return fail(FATTN_EWORKSPACE, std::string(who) + ": the backward needs a 256-byte aligned " +
                                      "workspace of at least " + std::to_string(l.bytes_min) +
                                      " bytes");
  }
  char* base = static_cast<char*>(ws);
  out->dsum = reinterpret_cast<float*>(base + l.d_off);
  out->part = ws_bytes >= l.bytes_split ? reinterpret_cast<float*>(base + l.part_off) : nullptr;
  out->arrive =
      out->part ? reinterpret_cast<unsigned long long*>(base + l.arrive_off) : nullptr;
  out->done = out->part ? reinterpret_cast<unsigned long long*>(base + l.done_off) : nullptr;
  out->epoch = out->part ? reinterpret_cast<unsigned long long*>(base + l.epoch_off) : nullptr;
  out->turn = reinterpret_cast<int*>(base + l.turn_off);
  out->ctrl = reinterpret_cast<int*>(base + l.ctrl_off);
  return 0;
}

int run_bwd_prep(const char* who, const float* o, View d_o, void* ws, size_t ws_bytes, int64_t b,
                 int64_t h, int64_t s, int64_t d, void* stream) {
  if (int rc = check_range(who, b, h, s, d)) return rc;
  if (!o || !d_o.p) return fail(FATTN_EINVAL, std::string(who) + ": null operand");
  if (!aligned16(o) || !view_aligned(d_o)) {
    return fail(FATTN_EALIGN, std::string(who) + ": rows must be 16-byte aligned");
  }
  WsParts p{};
  if (int rc = workspace_parts(who, ws, ws_bytes, b, h, s, d, &p)) return rc;
  // split (d <= 64, and d 128 with few key blocks per (b, h)): step 2 computes D itself and its
  // dQ sums need no clearing (epochs).
  if (!fattn::bwd_needs_prep(p.part != nullptr, static_cast<int>(d), s)) return ok();
  const int err = fattn::launch_bwd_prep(o, d_o, p.dsum, p.turn, p.ctrl, static_cast<int>(b),
                                         static_cast<int>(h), static_cast<int>(s),
                                         static_cast<int>(d), stream);
  if (err) return hip_fail(err, "backward step 1 launch");
  return ok();
}

// Step 2's operand checks (nothing launched).
int check_bwd_main(const char* who, View q, View k, View v, const float* o, View d_o,
                   const float* lse, float* dqkv, int64_t b, int64_t h, int64_t s, int64_t d) {
  if (int rc = check_range(who, b, h, s, d)) return rc;
  if (!slice_fits(q, s, d) || !slice_fits(k, s, d) || !slice_fits(v, s, d) ||
      !slice_fits(d_o, s, d) || s * 3 * h * d > int64_t{UINT32_MAX}) {
    return slice_error(who, s);
  }
  if (!q.p || !k.p || !v.p || !o || !d_o.p || !lse || !dqkv) {
    return fail(FATTN_EINVAL, std::string(who) + ": null operand");
  }
  if (!view_aligned(q) || !view_aligned(k) || !view_aligned(v) || !view_aligned(d_o) ||
      !aligned16(o) || !aligned16(dqkv)) {
    return fail(FATTN_EALIGN, std::string(who) + ": rows must be 16-byte aligned");
  }
  return 0;
}

int run_bwd_main(const char* who, View q, View k, View v, const float* o, View d_o,
                 const float* lse, float* dqkv, void* ws, size_t ws_bytes, int64_t b, int64_t h,
                 int64_t s, int64_t d, float scale, int causal, void* stream,
                 bool sums_final = false) {
  if (int rc = check_bwd_main(who, q, k, v, o, d_o, lse, dqkv, b, h, s, d)) return rc;
  WsParts p{};
  if (int rc = workspace_parts(who, ws, ws_bytes, b, h, s, d, &p)) return rc;
  const int err = fattn::launch_bwd_main(q, k, v, d_o, o, lse, p.dsum, dqkv, p.part, p.arrive,
                                         p.done, p.epoch, next_epoch(), p.turn, p.ctrl,
                                         static_cast<int>(b), static_cast<int>(h),
                                         static_cast<int>(s), static_cast<int>(d), scale,
                                         causal ? 1 : 0, 0, static_cast<int>(b * h),
                                         sums_final ? 1 : 0, stream);
  if (err) return hip_fail(err, "backward step 2 launch");
  return ok();
}

// Whether `stream` is capturing a HIP graph (or that cannot be told): then step 3 runs after
// step 2 even where step 2 sums every tile, because it also clears the sums' flags, which a
// replay of the graph (the same epoch) needs.
bool capturing(void* stream) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(static_cast<hipStream_t>(stream), &st) != hipSuccess) return true;
  return st != hipStreamCaptureStatusNone;
}

// Step 3: in split mode (the workspace holds the partials) dQ from the partials; else nothing.
int run_bwd_dq(const char* who, float* dqkv, void* ws, size_t ws_bytes, int64_t b, int64_t h,
               int64_t s, int64_t d, float scale, int causal, void* stream) {
  if (int rc = check_range(who, b, h, s, d)) return rc;
  if (s * 3 * h * d > int64_t{UINT32_MAX}) return slice_error(who, s);
  if (!dqkv) return fail(FATTN_EINVAL, std::string(who) + ": null operand");
  if (!aligned16(dqkv)) {
    return fail(FATTN_EALIGN, std::string(who) + ": rows must be 16-byte aligned");
  }
  WsParts p{};
  if (int rc = workspace_parts(who, ws, ws_bytes, b, h, s, d, &p)) return rc;
  if (!p.part) return ok();
  const int err = fattn::launch_bwd_dq(p.part, p.done, p.arrive, p.epoch, dqkv,
                                       static_cast<int>(b), static_cast<int>(h),
                                       static_cast<int>(s), static_cast<int>(d), scale,
                                       causal ? 1 : 0, 0, static_cast<int>(b * h), stream);
  if (err) return hip_fail(err, "backward step 3 launch");
  return ok();
}

// Steps 2 and 3 of the split sum over the (b, h) in chunks of `chunk` pairs, each chunk's
// partials, arrival slots and done flags at the start of the workspace (no step 1 at d <= 64).
int run_backward_chunked(const char* who, View q, View k, View v, const float* o, View d_o,
                         const float* lse, float* dqkv, void* ws, size_t ws_bytes, int64_t b,
                         int64_t h, int64_t s, int64_t d, float scale, int causal, int64_t chunk,
                         void* stream) {
  if (int rc = check_bwd_main(who, q, k, v, o, d_o, lse, dqkv, b, h, s, d)) return rc;
  WsParts p{};
  if (int rc = workspace_parts(who, ws, ws_bytes, 1, chunk, s, d, &p)) return rc;
  if (!p.part) return fail(FATTN_EWORKSPACE, std::string(who) + ": workspace too small");
  const bool eager = !capturing(stream);
  for (int64_t bh0 = 0; bh0 < b * h; bh0 += chunk) {
    const int n = static_cast<int>(std::min(chunk, b * h - bh0));
    const bool final_sums =
        eager && fattn::bwd_step2_sums_all(n, b, h, s, static_cast<int>(d), causal ? 1 : 0);
    int err = fattn::launch_bwd_main(q, k, v, d_o, o, lse, p.dsum, dqkv, p.part, p.arrive, p.done,
                                     p.epoch, next_epoch(), p.turn, p.ctrl, static_cast<int>(b),
                                     static_cast<int>(h), static_cast<int>(s),
                                     static_cast<int>(d), scale, causal ? 1 : 0,
                                     static_cast<int>(bh0), n, final_sums ? 1 : 0, stream);
    if (err) return hip_fail(err, "backward step 2 launch");
    if (final_sums) continue;
    err = fattn::launch_bwd_dq(p.part, p.done, p.arrive, p.epoch, dqkv, static_cast<int>(b),
                               static_cast<int>(h), static_cast<int>(s), static_cast<int>(d),
                               scale, causal ? 1 : 0, static_cast<int>(bh0), n, stream);
    if (err) return hip_fail(err, "backward step 3 launch");
  }
  return ok();
}

int run_backward(const char* who, View q, View k, View v, const float* o, View d_o,
                 const float* lse, float* dqkv, void* ws, size_t ws_bytes, int64_t b, int64_t h,
                 int64_t s, int64_t d, float scale, int causal, void* stream) {
  // A workspace that holds the split sum of some (b, h) but not of all: the split sum by chunks
  // where the chunks are large enough to beat the turn hand-over (or the workspace is too small
  // for the turn hand-over's minimum).
  if (int rc = check_range(who, b, h, s, d)) return rc;
  int64_t chunk = 0;
  if (ws) {
    chunk = fattn::split_chunk(b, h, s, d, ws_bytes,
                               fattn::min_chunk_pairs(b, h, s, d, causal != 0), causal != 0);
    if (chunk == 0 && ws_bytes < fattn::workspace_layout(b, h, s, d).bytes_min) {
      chunk = fattn::split_chunk(b, h, s, d, ws_bytes, 1, causal != 0);
    }
  }
  if (chunk > 0 && chunk < b * h) {
    return run_backward_chunked(who, q, k, v, o, d_o, lse, dqkv, ws, ws_bytes, b, h, s, d, scale,
                                causal, chunk, stream);
  }
  if (int rc = run_bwd_prep(who, o, d_o, ws, ws_bytes, b, h, s, d, stream)) return rc;
  // Step 3 only where step 2's sums may leave tiles (or a graph is being captured).
  const bool final_sums = ws && ws_bytes >= fattn::workspace_layout(b, h, s, d).bytes_split &&
                          fattn::bwd_step2_sums_all(b * h, b, h, s, static_cast<int>(d),
                                                    causal ? 1 : 0) &&
                          !capturing(stream);
  if (int rc = run_bwd_main(who, q, k, v, o, d_o, lse, dqkv, ws, ws_bytes, b, h, s, d, scale,
                            causal, stream, final_sums)) {
    return rc;
  }
  if (final_sums) return ok();
  return run_bwd_dq(who, dqkv, ws, ws_bytes, b, h, s, d, scale, causal, stream);
}

bool negative(const int64_t* x, int n) {
  for (int i = 0; i < n; ++i) {
    if (x[i] < 0) return true;
  }
  return false;
}

// qkv_geometry (src/lib.rs:191-206): dims (b, heads, s, d); q / k / v view strides
// [sb, d, ss] at element offsets 0, h d, 2 h d.
int qkv_geometry(const int64_t shape[3], const int64_t strides[3], int64_t heads, int64_t* b,
                 int64_t* s, int64_t* d) {
  if (!shape || !strides || negative(shape, 3) || negative(strides, 3)) {
    return fail(FATTN_EINVAL, "fused_attention_qkv: a [b, s, 3 h d] layout expected");
  }
  const int64_t three_hd = shape[2];
  if (heads <= 0 || three_hd % (3 * heads) != 0) {
    return fail(FATTN_EINVAL, "fused_attention_qkv: last dimension " + std::to_string(three_hd) +
                                  " is not 3 x " + std::to_string(heads) +
                                  " heads x head_dim");
  }
  if (strides[2] != 1 && three_hd > 1) {
    return fail(FATTN_EINVAL,
                "fused_attention_qkv: the last dimension must be contiguous, strides " +
                    dims_str(strides, 3));
  }
  *b = shape[0];
  *s = shape[1];
  *d = three_hd / 3 / heads;
  return 0;
}

// check_shapes + bhs_strides (src/lib.rs:181-220) over q, k, v.
int bhsd_geometry(const int64_t* qs, const int64_t* qst, const int64_t* ks, const int64_t* kst,
                  const int64_t* vs, const int64_t* vst) {
  if (!qs || !qst || !ks || !kst || !vs || !vst || negative(qs, 4) || negative(qst, 4) ||
      negative(ks, 4) || negative(kst, 4) || negative(vs, 4) || negative(vst, 4)) {
    return fail(FATTN_EINVAL, "fused_attention: a [b, h, s, d] layout expected");
  }
  for (int i = 0; i < 4; ++i) {
    if (ks[i] != qs[i] || vs[i] != qs[i]) {
      return fail(FATTN_EINVAL, "fused_attention: q, k, v must share one [b, h, s, d] shape, got " +
                                    dims_str(qs, 4) + " " + dims_str(ks, 4) + " " +
                                    dims_str(vs, 4));
    }
  }
  const int64_t* all[3] = {qst, kst, vst};
  for (const int64_t* st : all) {
    if (st[3] != 1 && qs[3] > 1) {
      return fail(FATTN_EINVAL,
                  "fused_attention: [b, h, s, d] with d contiguous expected, strides " +
                      dims_str(st, 4));
    }
  }
  return 0;
}

bool empty3(int64_t b, int64_t h, int64_t s) { return b == 0 || h == 0 || s == 0; }

}  // namespace

extern "C" {

const char* fattn_last_error(void) { return g_error.c_str(); }

const char* fattn_version(void) {
  return "fattn-gfx950 0.2.0 (head_dim 32, 64, 128; fp32 MFMA)";
}

size_t fattn_bwd_workspace_bytes(int64_t b, int64_t h, int64_t s, int64_t d) {
  if (b < 0 || h < 0 || s < 0 || !fattn::head_dim_supported(d)) return 0;
  return fattn::workspace_within(b, h, s, d, FATTN_SPLIT_MAX_BYTES);
}

size_t fattn_bwd_workspace_min_bytes(int64_t b, int64_t h, int64_t s, int64_t d) {
  if (b < 0 || h < 0 || s < 0 || !fattn::head_dim_supported(d)) return 0;
  return fattn::workspace_layout(b, h, s, d).bytes_min;
}

size_t fattn_bwd_workspace_split_bytes(int64_t b, int64_t h, int64_t s, int64_t d) {
  if (b < 0 || h < 0 || s < 0 || !fattn::head_dim_supported(d)) return 0;
  return fattn::workspace_layout(b, h, s, d).bytes_split;
}

int fattn_fwd_f32(const float* q, const float* k, const float* v, float* o, float* lse, int64_t b,
                  int64_t h, int64_t s, int64_t d, float scale, int causal,
                  const int64_t q_strides[3], const int64_t k_strides[3],
                  const int64_t v_strides[3], void* stream) {
  if (b < 0 || h < 0 || s < 0) return fail(FATTN_EINVAL, "fused_attention: negative size");
  if (int rc = check_head_dim(d)) return rc;
  if (empty3(b, h, s)) return ok();
  if (!q_strides || !k_strides || !v_strides) {
    return fail(FATTN_EINVAL, "fused_attention: null strides");
  }
  return run_forward("fused_attention", make_view(q, q_strides), make_view(k, k_strides),
                     make_view(v, v_strides), o, lse, b, h, s, d, scale, causal, stream);
}

int fattn_bwd_prep_f32(const float* o, const float* d_o, const int64_t do_strides[3],
                       void* workspace, size_t workspace_bytes, int64_t b, int64_t h, int64_t s,
                       int64_t d, void* stream) {
  if (b < 0 || h < 0 || s < 0) return fail(FATTN_EINVAL, "fused_attention: negative size");
  if (int rc = check_head_dim(d)) return rc;
  if (empty3(b, h, s)) return ok();
  if (!do_strides) return fail(FATTN_EINVAL, "fused_attention: null strides");
  return run_bwd_prep("fused_attention", o, make_view(d_o, do_strides), workspace,
                      workspace_bytes, b, h, s, d, stream);
}

int fattn_bwd_main_f32(const float* q, const float* k, const float* v, const float* o,
                       const float* d_o, const float* lse, float* dqkv, void* workspace,
                       size_t workspace_bytes, int64_t b, int64_t h, int64_t s, int64_t d,
                       float scale, int causal, const int64_t q_strides[3],
                       const int64_t k_strides[3], const int64_t v_strides[3],
                       const int64_t do_strides[3], void* stream) {
  if (b < 0 || h < 0 || s < 0) return fail(FATTN_EINVAL, "fused_attention: negative size");
  if (int rc = check_head_dim(d)) return rc;
  if (empty3(b, h, s)) return ok();
  if (!q_strides || !k_strides || !v_strides || !do_strides) {
    return fail(FATTN_EINVAL, "fused_attention: null strides");
  }
  return run_bwd_main("fused_attention", make_view(q, q_strides), make_view(k, k_strides),
                      make_view(v, v_strides), o, make_view(d_o, do_strides), lse, dqkv,
                      workspace, workspace_bytes, b, h, s, d, scale, causal, stream);
}

int fattn_bwd_dq_f32(float* dqkv, void* workspace, size_t workspace_bytes, int64_t b, int64_t h,
                     int64_t s, int64_t d, float scale, int causal, void* stream) {
  if (b < 0 || h < 0 || s < 0) return fail(FATTN_EINVAL, "fused_attention: negative size");
  if (int rc = check_head_dim(d)) return rc;
  if (empty3(b, h, s)) return ok();
  return run_bwd_dq("fused_attention", dqkv, workspace, workspace_bytes, b, h, s, d, scale,
                    causal, stream);
}

int fattn_bwd_f32(const float* q, const float* k, const float* v, const float* o,
                  const float* d_o, const float* lse, float* dqkv, void* workspace,
                  size_t workspace_bytes, int64_t b, int64_t h, int64_t s, int64_t d,
                  float scale, int causal, const int64_t q_strides[3],
                  const int64_t k_strides[3], const int64_t v_strides[3],
                  const int64_t do_strides[3], void* stream) {
  if (b < 0 || h < 0 || s < 0) return fail(FATTN_EINVAL, "fused_attention: negative size");
  if (int rc = check_head_dim(d)) return rc;
  if (empty3(b, h, s)) return ok();
  if (!q_strides || !k_strides || !v_strides || !do_strides) {
    return fail(FATTN_EINVAL, "fused_attention: null strides");
  }
  return run_backward("fused_attention", make_view(q, q_strides), make_view(k, k_strides),
                      make_view(v, v_strides), o, make_view(d_o, do_strides), lse, dqkv,
                      workspace, workspace_bytes, b, h, s, d, scale, causal, stream);
}

int fattn_bwd_f32_noalloc(const float* q, const float* k, const float* v, const float* o,
                          const float* d_o, const float* lse, float* dqkv, int64_t b, int64_t h,
                          int64_t s, int64_t d, float scale, int causal,
                          const int64_t q_strides[3], const int64_t k_strides[3],
                          const int64_t v_strides[3], const int64_t do_strides[3], void* stream) {
  const char* who = "fused_attention";
  if (b < 0 || h < 0 || s < 0) return fail(FATTN_EINVAL, "fused_attention: negative size");
  if (int rc = check_head_dim(d)) return rc;
  if (empty3(b, h, s)) return ok();
  if (!q_strides || !k_strides || !v_strides || !do_strides) {
    return fail(FATTN_EINVAL, "fused_attention: null strides");
  }
  if (int rc = check_range(who, b, h, s, d)) return rc;
  // dQ summed as fattn_bwd_f32 sums it with a workspace of the scratch's size: the whole split
  // when it fits, else (d <= 64) the split by chunks of (b, h) pairs, else the turn hand-over.
  const size_t need = fattn::workspace_within(b, h, s, d, FATTN_STATIC_SCRATCH_BYTES);
  if (need > FATTN_STATIC_SCRATCH_BYTES) {
    return fail(FATTN_EWORKSPACE,
                std::string(who) + ": the backward of " + std::to_string(b) + " x " +
                    std::to_string(h) + " x " + std::to_string(s) + " needs a workspace of " +
                    std::to_string(need) + " bytes; the static scratch holds " +
                    std::to_string(FATTN_STATIC_SCRATCH_BYTES) +
                    " (pass a workspace to fattn_bwd_f32)");
  }
  void* ws = nullptr;
  if (int err = fattn::static_scratch(stream, &ws)) return hip_fail(err, "static scratch");
  return run_backward(who, make_view(q, q_strides), make_view(k, k_strides),
                      make_view(v, v_strides), o, make_view(d_o, do_strides), lse, dqkv, ws, need,
                      b, h, s, d, scale, causal, stream);
}

// The reference-named head_dim-64 entries: the generic ones behind the reference's check.
int fattn_fwd_f32_d64(const float* q, const float* k, const float* v, float* o, float* lse,
                      int64_t b, int64_t h, int64_t s, int64_t d, float scale, int causal,
                      const int64_t q_strides[3], const int64_t k_strides[3],
                      const int64_t v_strides[3], void* stream) {
  if (int rc = check_head_dim64(d)) return rc;
  return fattn_fwd_f32(q, k, v, o, lse, b, h, s, d, scale, causal, q_strides, k_strides,
                       v_strides, stream);
}

int fattn_bwd_prep_f32_d64(const float* o, const float* d_o, const int64_t do_strides[3],
                           void* workspace, size_t workspace_bytes, int64_t b, int64_t h,
                           int64_t s, int64_t d, void* stream) {
  if (int rc = check_head_dim64(d)) return rc;
  return fattn_bwd_prep_f32(o, d_o, do_strides, workspace, workspace_bytes, b, h, s, d, stream);
}

int fattn_bwd_main_f32_d64(const float* q, const float* k, const float* v, const float* o,
                           const float* d_o, const float* lse, float* dqkv, void* workspace,
                           size_t workspace_bytes, int64_t b, int64_t h, int64_t s, int64_t d,
                           float scale, int causal, const int64_t q_strides[3],
                           const int64_t k_strides[3], const int64_t v_strides[3],
                           const int64_t do_strides[3], void* stream) {
  if (int rc = check_head_dim64(d)) return rc;
  return fattn_bwd_main_f32(q, k, v, o, d_o, lse, dqkv, workspace, workspace_bytes, b, h, s, d,
                            scale, causal, q_strides, k_strides, v_strides, do_strides, stream);
}

int fattn_bwd_dq_f32_d64(float* dqkv, void* workspace, size_t workspace_bytes, int64_t b,
                         int64_t h, int64_t s, int64_t d, float scale, int causal, void* stream) {
  if (int rc = check_head_dim64(d)) return rc;
  return fattn_bwd_dq_f32(dqkv, workspace, workspace_bytes, b, h, s, d, scale, causal, stream);
}

int fattn_bwd_f32_d64(const float* q, const float* k, const float* v, const float* o,
                      const float* d_o, const float* lse, float* dqkv, void* workspace,
                      size_t workspace_bytes, int64_t b, int64_t h, int64_t s, int64_t d,
                      float scale, int causal, const int64_t q_strides[3],
                      const int64_t k_strides[3], const int64_t v_strides[3],
                      const int64_t do_strides[3], void* stream) {
  if (int rc = check_head_dim64(d)) return rc;
  return fattn_bwd_f32(q, k, v, o, d_o, lse, dqkv, workspace, workspace_bytes, b, h, s, d, scale,
                       causal, q_strides, k_strides, v_strides, do_strides, stream);
}

int fattn_qkv_forward(const float* qkv, int64_t offset, const int64_t shape[3],
                      const int64_t strides[3], int64_t heads, float scale, int causal,
                      float* out, float* lse, void* stream) {
  int64_t b = 0, s = 0, d = 0;
  if (int rc = qkv_geometry(shape, strides, heads, &b, &s, &d)) return rc;
  if (int rc = check_head_dim(d)) return rc;
  if (empty3(b, heads, s)) return ok();
  if (!qkv || offset < 0) return fail(FATTN_EINVAL, "fused_attention_qkv: null operand");
  const int64_t hd = heads * d;
  const float* base = qkv + offset;
  if (!aligned16(base) || strides[0] % 4 != 0 || strides[1] % 4 != 0) {
    return fail(FATTN_EALIGN, "fused_attention_qkv: rows must be 16-byte aligned");
  }
  const View q{base, strides[0], d, strides[1]};
  const View k{base + hd, strides[0], d, strides[1]};
  const View v{base + 2 * hd, strides[0], d, strides[1]};
  return run_forward("fused_attention_qkv", q, k, v, out, lse, b, heads, s, d, scale, causal,
                     stream);
}

int fattn_qkv_backward(const float* qkv, int64_t offset, const int64_t shape[3],
                       const int64_t strides[3], int64_t heads, float scale, int causal,
                       const float* out, const float* lse, const float* grad,
                       int64_t grad_offset, const int64_t grad_shape[3],
                       const int64_t grad_strides[3], float* dqkv, void* workspace,
                       size_t workspace_bytes, void* stream) {
  int64_t b = 0, s = 0, d = 0;
  if (int rc = qkv_geometry(shape, strides, heads, &b, &s, &d)) return rc;
  if (int rc = check_head_dim(d)) return rc;
  const int64_t hd = heads * d;
  if (!grad_shape || !grad_strides || grad_shape[0] != b || grad_shape[1] != s ||
      grad_shape[2] != hd) {
    const int64_t want[3] = {b, s, hd};
    return fail(FATTN_EINVAL, "fused_attention_qkv: rank-3 gradient of shape " +
                                  dims_str(want, 3) + " expected");
  }
  if (grad_strides[2] != 1 && hd > 1) {
    return fail(FATTN_EINVAL, "fused_attention_qkv: the gradient's last dimension must be "
                              "contiguous, strides " + dims_str(grad_strides, 3));
  }
  if (empty3(b, heads, s)) return ok();
  if (!qkv || !grad || offset < 0 || grad_offset < 0) {
    return fail(FATTN_EINVAL, "fused_attention_qkv: null operand");
  }
  const float* base = qkv + offset;
  if (!aligned16(base) || strides[0] % 4 != 0 || strides[1] % 4 != 0) {
    return fail(FATTN_EALIGN, "fused_attention_qkv: rows must be 16-byte aligned");
  }
  const View q{base, strides[0], d, strides[1]};
  const View k{base + hd, strides[0], d, strides[1]};
  const View v{base + 2 * hd, strides[0], d, strides[1]};
  const View g{grad + grad_offset, grad_strides[0], d, grad_strides[1]};
  return run_backward("fused_attention_qkv", q, k, v, out, g, lse, dqkv, workspace,
                      workspace_bytes, b, heads, s, d, scale, causal, stream);
}

int fattn_forward(const float* q, int64_t q_offset, const int64_t q_shape[4],
                  const int64_t q_strides[4], const float* k, int64_t k_offset,
                  const int64_t k_shape[4], const int64_t k_strides[4], const float* v,
                  int64_t v_offset, const int64_t v_shape[4], const int64_t v_strides[4],
                  float scale, int causal, float* out, float* lse, void* stream) {
  if (int rc = bhsd_geometry(q_shape, q_strides, k_shape, k_strides, v_shape, v_strides)) {
    return rc;
  }
  if (int rc = check_head_dim(q_shape[3])) return rc;
  const int64_t b = q_shape[0], h = q_shape[1], s = q_shape[2], d = q_shape[3];
  if (empty3(b, h, s)) return ok();
  if (!q || !k || !v || q_offset < 0 || k_offset < 0 || v_offset < 0) {
    return fail(FATTN_EINVAL, "fused_attention: null operand");
  }
  const View qv{q + q_offset, q_strides[0], q_strides[1], q_strides[2]};
  const View kv{k + k_offset, k_strides[0], k_strides[1], k_strides[2]};
  const View vv{v + v_offset, v_strides[0], v_strides[1], v_strides[2]};
  return run_forward("fused_attention", qv, kv, vv, out, lse, b, h, s, d, scale, causal, stream);
}

int fattn_backward(const float* q, int64_t q_offset, const int64_t q_shape[4],
                   const int64_t q_strides[4], const float* k, int64_t k_offset,
                   const int64_t k_shape[4], const int64_t k_strides[4], const float* v,
                   int64_t v_offset, const int64_t v_shape[4], const int64_t v_strides[4],
                   float scale, int causal, const float* out, const float* lse,
                   const float* grad, int64_t grad_offset, const int64_t grad_shape[4],
                   const int64_t grad_strides[4], float* dqkv, void* workspace,
                   size_t workspace_bytes, void* stream) {
  if (int rc = bhsd_geometry(q_shape, q_strides, k_shape, k_strides, v_shape, v_strides)) {
    return rc;
  }
  if (int rc = check_head_dim(q_shape[3])) return rc;
  const int64_t b = q_shape[0], h = q_shape[1], s = q_shape[2], d = q_shape[3];
  // The gradient of the [b, s, h, d] raw output (src/lib.rs:465-475: strides [gb, gs, gh, 1]).
  if (!grad_shape || !grad_strides || grad_shape[0] != b || grad_shape[1] != s ||
      grad_shape[2] != h || grad_shape[3] != d) {
    return fail(FATTN_EINVAL, "fused_attention: rank-4 gradient expected");
  }
  if (grad_strides[3] != 1 && d > 1) {
    return fail(FATTN_EINVAL,
                "fused_attention: the gradient's last dimension must be contiguous, strides " +
                    dims_str(grad_strides, 4));
  }
  if (empty3(b, h, s)) return ok();
  if (!q || !k || !v || !grad || q_offset < 0 || k_offset < 0 || v_offset < 0 ||
      grad_offset < 0) {
    return fail(FATTN_EINVAL, "fused_attention: null operand");
  }
  const View qv{q + q_offset, q_strides[0], q_strides[1], q_strides[2]};
  const View kv{k + k_offset, k_strides[0], k_strides[1], k_strides[2]};
  const View vv{v + v_offset, v_strides[0], v_strides[1], v_strides[2]};
  const View g{grad + grad_offset, grad_strides[0], grad_strides[2], grad_strides[1]};
  return run_backward("fused_attention", qv, kv, vv, out, g, lse, dqkv, workspace,
                      workspace_bytes, b, h, s, d, scale, causal, stream);
}

// Test hook (not declared in include/fattn.h; tests/test_boundary.py calls it without a GPU): an
// audit of step 2's dQ-sum schedule for one shape, on the host, with the scheduling functions the
// kernel runs (fattn_internal.h). A summing unit is a workgroup appended to step 2's grid
// (non-causal) or a key block's own workgroup summing its diagonal tiles (causal). out[0]:
// workgroups appended to step 2's grid; out[1]: summing units with tiles to sum; out[2]:
// violations -- a causal unit waits for a key block later in the grid or sums a tile it is not
// the last contributor of, a non-causal unit of XCD x takes a (b, h) whose last key block
// xcd_remap does not put on x (or, past the XCDs' ranges, one that is not dealt round robin),
// xcd_remap and item_xcd disagree, or a workgroup past the plan's range has a target; out[3]: query tiles two units would both sum;
// out[4]: query tiles summed; out[5]: keys per key block (bwd_split_keys).
int fattn_internal_sum_audit(int64_t b, int64_t h, int64_t s, int64_t d, int causal,
                             int64_t out[6]) {
  if (!out || b <= 0 || h <= 0 || s <= 0 || b * h * s > (int64_t{1} << 26)) return FATTN_EINVAL;
  const int BH = static_cast<int>(b * h);
  const int keys = fattn::bwd_split_keys(b, h, s, static_cast<int>(d), causal);
  const int nkb = static_cast<int>((s + keys - 1) / keys);
  const int ntile = static_cast<int>((s + fattn::kBwdQueryTile - 1) / fattn::kBwdQueryTile);
  const int total = nkb * BH;
  const fattn::SumPlan plan = fattn::sum_plan(BH, nkb, ntile, static_cast<int>(d), causal);
  const int64_t nsum = fattn::bwd_sum_blocks(b, h, s, static_cast<int>(d), causal);
  const bool sums = fattn::bwd_step2_sums(b, h, s, static_cast<int>(d), causal);
  int64_t targets = 0, bad = 0, twice = 0, covered = 0;
  // xcd_remap is a permutation and item_xcd its inverse's XCD.
  std::vector<char> seen(static_cast<size_t>(total), 0);
  for (int id = 0; id < total; ++id) {
    const int item = fattn::xcd_remap(id, total);
    if (item < 0 || item >= total || seen[item]++ || fattn::item_xcd(item, total) != (id & 7)) {
      ++bad;
    }
  }
  // The key blocks a unit summing tiles j0 .. j1 - 1 waits for: all, or (causal) those holding a
  // key <= its last query.
  auto need_of = [&](int j1) {
    return causal ? static_cast<int>(std::min<int64_t>(nkb - 1, std::min<int64_t>(s - 1,
                        int64_t{j1} * fattn::kBwdQueryTile - 1) / keys)) + 1
                  : nkb;
  };
  std::vector<char> tile_done(static_cast<size_t>(BH) * ntile, 0);
  auto mark = [&](int bh, int j0, int j1) {
    for (int j = j0; j < j1; ++j) {
      if (tile_done[static_cast<size_t>(bh) * ntile + j]++) ++twice;
      ++covered;
    }
  };
  if (causal) {
    if (nsum != 0) ++bad;
    // Key block kb of (b, h) bh is workgroup kb b h + bh (no remap).
    for (int bh = 0; sums && bh < BH; ++bh) {
      for (int kb = 0; kb < nkb; ++kb) {
        int j0 = 0, j1 = 0;
        fattn::own_tiles(kb, keys, ntile, &j0, &j1);
        if (j0 >= j1) continue;
        ++targets;
        const int id = kb * BH + bh, need = need_of(j1);
        if (need != kb + 1 || need_of(j0 + 1) != kb + 1) ++bad;  // not its last contributor
        for (int k = 0; k < need; ++k) {
          if (k * BH + bh > id) ++bad;  // a contributor later in the grid
        }
        mark(bh, j0, j1);
      }
    }
  } else {
    for (int64_t i = 0; i < nsum + 64; ++i) {  // 64 past the grid: nothing may be assigned there
      const int x = static_cast<int>(i & 7), m = static_cast<int>(i >> 3);
      int bh = -1, j0 = -1;
      if (!fattn::sum_target(plan, x, m, BH, causal, &bh, &j0)) continue;
      if (i >= nsum || bh < 0 || bh >= BH || j0 < 0 || j0 >= ntile) {
        ++bad;
        continue;
      }
      ++targets;
      const int j1 = std::min(ntile, j0 + fattn::kSumTiles);
      // Key block kb of (b, h) bh: the (b, h)-major item bh nkb + kb under xcd_remap; summing
      // workgroups come after every key block in the grid. The first mc nchunk of each XCD take
      // (b, h)s whose last key block runs on that XCD, the rest (b, h)s whose last key block is
      // one of those dealt round robin.
      const int last = bh * nkb + nkb - 1;
      if (m < plan.mc * plan.nchunk ? fattn::item_xcd(last, total) != x
                                    : last < (total & ~7)) {
        ++bad;
      }
      mark(bh, j0, j1);
    }
  }
  out[0] = nsum;
  out[1] = targets;
  out[2] = bad;
  out[3] = twice;
  out[4] = covered;
  out[5] = keys;
  return 0;
}

// The test hooks below change how every later backward of the process runs. They act only in a
// process that opted in before the library loaded (FATTN_TEST_HOOKS=1 in its environment, read
// once, at load); otherwise they change nothing and return FATTN_EINVAL.

// Test hook (not declared in include/fattn.h): step 2's dQ sums on (1, the default) or off (0:
// step 3 sums every tile) for every later backward of the process. Returns the previous setting.
int fattn_internal_step2_sums(int on) {
  if (!g_test_hooks) return hooks_refused("fattn_internal_step2_sums");
  return fattn::set_step2_sums(on != 0) ? 1 : 0;
}

// Test hook (not declared in include/fattn.h): step 2's non-causal summing workgroups of XCD x
// sum the (b, h)s whose key blocks ran on XCD x + shift (mod 8) in every later backward of the
// process (0, the default: their own XCD's), so that a test can make every sum read partials
// written on another XCD. Returns the previous shift.
int fattn_internal_sum_shift(int shift) {
  if (!g_test_hooks) return hooks_refused("fattn_internal_sum_shift");
  return fattn::set_sum_shift(shift);
}

// Test hook (not declared in include/fattn.h): the dQ sums of (b, h) pair `bh` (index b * h_count
// + h; -1, the default: none) give up before their first poll in every later backward of the
// process, as a wait that timed out would: where no step 3 follows they raise the guard word (3)
// and write NaN into that pair's dQ rows; where step 3 follows it sums them. Returns the previous
// pair.
int fattn_internal_sum_give_up(int bh) {
  if (!g_test_hooks) return hooks_refused("fattn_internal_sum_give_up");
  return fattn::set_give_up_bh(bh);
}

// Test hook (not declared in include/fattn.h; read-only, always allowed): the hooks' current
// settings, out[0] step 2's sums on, out[1] the sum shift, out[2] the give-up pair; returns 1 if
// the hooks may act in this process, else 0.
int fattn_internal_hooks(int64_t out[3]) {
  if (!out) return FATTN_EINVAL;
  fattn::test_hook_state(out);
  return g_test_hooks ? 1 : 0;
}

int fattn_bwd_status(const void* workspace, size_t workspace_bytes, int64_t b, int64_t h,
                     int64_t s, void* stream, int* status) {
  if (!status) return fail(FATTN_EINVAL, "fused_attention: null status");
  *status = 0;
  if (b < 0 || h < 0 || s < 0) return fail(FATTN_EINVAL, "fused_attention: negative size");
  // The control words open every workspace layout (whole, chunked, minimum): the guard word's
  // place depends on nothing else.
  if (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 255u) != 0 ||
      workspace_bytes < 64 * sizeof(int)) {
    return fail(FATTN_EWORKSPACE, "fused_attention: the backward needs a 256-byte aligned "
                                  "workspace of at least 256 bytes");
  }
  hipError_t err = hipStreamSynchronize(static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return hip_fail(err, "status sync");
  int guard = 0;
  err = hipMemcpy(&guard, static_cast<const int*>(workspace) + fattn::kCtrlGuard, sizeof(int),
                  hipMemcpyDeviceToHost);
  if (err != hipSuccess) return hip_fail(err, "status copy");
  *status = guard;
  return ok();
}

}  // extern "C"
