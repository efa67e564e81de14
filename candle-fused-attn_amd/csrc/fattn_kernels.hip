// Fused fp32 scaled-dot-product attention for gfx950 (MI355X / CDNA4), head_dim D = 32, 64 or 128
// (every kernel is a template on D; 64 is the reference's, 32 and 128 its roadmap's): a
// FlashAttention-2-style forward (online softmax, the [s, s] scores never written, only O and the
// row log-sum-exp L stored) and a deterministic one-pass backward.
//
// Every product runs on the fp32 matrix cores: v_mfma_f32_16x16x4_f32 (true fp32 inputs, fp32
// accumulate). For one instruction, lane l (lo = l % 16, g = l / 16) supplies A[lo][g] and B[g][lo]
// of a 16x4 by 4x16 product and holds D[4 g + r][lo], r = 0..3. Three consequences shape the
// kernels:
//   - the contraction index of a step is (g, step), so any bijection from (g, step) to the
//     contracted dimension is allowed, as long as A and B use the same one;
//   - a product's output row index lives in (g, r) and its column index in lo, so a result can feed
//     the next product as its B operand (contraction over the rows) without moving: P = exp(S - L)
//     leaves S^T's accumulator and enters O^T = V^T P^T as is (forward); P and dS leave S's
//     accumulator and enter dV^T = dO^T P and dK^T = Q^T dS as is (backward);
//   - the forward's rows (queries) sit in lo, so the online-softmax state of a query is one lane's
//     (plus the three lanes lo + 16, + 32, + 48 holding its other keys): no cross-lane traffic
//     but one max exchange per tile.
//
// Layouts (element offsets; strides in floats): q, k, v and dO are read through (batch, head,
// seq) strides with head_dim contiguous, every row 16-byte aligned; O is written [b, s, h, D];
// L and D are [b, h, s]; dQ, dK, dV are written interleaved into one [b, s, 3, h, D] buffer.
//
// Determinism: every sum has an order fixed by the shape alone. The cross-workgroup sum (dQ over
// key blocks) is done one of two ways, chosen by the size of the caller's workspace:
//   split: every key block writes its dQ partial of each query tile to its own slot of the
//     workspace (no workgroup waits on another); a second kernel sums the slots in key-block
//     order, scales, and writes dQ;
//   turns: key blocks add into dQ in place, in an order fixed per tile, under one turn counter per
//     (b, h, query tile); key blocks are handed out by a ticket in arrival order, so a workgroup
//     only ever waits on a key block that a running workgroup already holds (no assumption about
//     dispatch order). Needs no workspace beyond D and the counters.
#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <stddef.h>
#include <stdint.h>

#include "fattn.h"
#include "fattn_internal.h"

// The backward workspace of fattn_bwd_f32_noalloc, for callers that cannot allocate: device memory
// of this library, one copy per GPU (each at its own address), held until the process ends. In
// host code the name is only a host-side handle: the device address comes from
// hipGetSymbolAddress (fattn::static_scratch below), never from the name itself.
static __device__ __align__(256) unsigned char scratch[FATTN_STATIC_SCRATCH_BYTES];

namespace fattn {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
// An int known at compile time, or not, behind the same call syntax.
template <int V>
struct Const {
  static constexpr int value = V;
  __device__ constexpr int operator()() const { return V; }
};
struct Var {
  int v;
  __device__ int operator()() const { return v; }
};

constexpr int kThreads = 256;  // 4 waves of 64
constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kNegInf = -__builtin_inff();
// Forward lazy rescaling: a row's reference max moves only when a tile's max exceeds it by more
// than this many powers of two (unnormalised probabilities stay below 2^8).
constexpr float kRescaleLog2 = 8.0f;
// A dQ turn wait gives up after this many polls (about a second) and raises the guard word,
// so a protocol failure ends the kernel instead of hanging the GPU.
constexpr int kSpinBound = 1 << 20;

__device__ __forceinline__ f4 mma(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
// 2^x on the transcendental unit (v_exp_f32); 2^-inf = 0.
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ f4 ld4(const float* p) { return *reinterpret_cast<const f4*>(p); }
__device__ __forceinline__ void st4(float* p, f4 v) { *reinterpret_cast<f4*>(p) = v; }
// Non-temporal store (nt): for outputs no kernel of the same pass reads again, so that they do not
// sit dirty in the L2s when the kernel ends (each XCD's L2 writes its dirty lines back then).
__device__ __forceinline__ void st4_nt(float* p, f4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<f4*>(p));
}
__device__ __forceinline__ f4 zero4() { return f4{0.0f, 0.0f, 0.0f, 0.0f}; }
// 16 bytes stored / loaded at device scope (cache-policy bit sc1: through to the coherence point
// that all XCDs share), as buffer accesses from a wave-uniform base that cover `bytes` bytes
// (accesses past them are dropped / read 0). The dQ partials and their sums in step 2 use them,
// so that a sum may read partials written by a key block on another XCD.
constexpr int kScDevice = 16;              // the buffer access's cache-policy operand: sc1
constexpr int kRsrcWord3 = 0x00020000;     // gfx9 buffer descriptor: 32-bit data format
typedef unsigned u4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dev_rsrc(const float* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, bytes, kRsrcWord3);
}
__device__ __forceinline__ void st4_dev(__amdgpu_buffer_rsrc_t r, unsigned off, f4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v), r, off, 0, kScDevice);
}
__device__ __forceinline__ f4 ld4_dev(__amdgpu_buffer_rsrc_t r, unsigned off) {
  return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kScDevice));
}

// A lane of x through a DPP lane permutation (VALU, no LDS round trip).
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
// Sum over each aligned group of N = 8, 16 or 32 lanes, every lane of the group getting the same
// bits (each step adds a lane and its partner, and x + y == y + x): partner = lane ^ 1
// (quad_perm 1,0,3,2), lane ^ 2 (quad_perm 2,3,0,1), the other quad of the 8 (row_half_mirror),
// the other 8 of the 16 (row_mirror), the other 16 of the 32 (row swap).
template <int N>
__device__ __forceinline__ float lane_sum(float x) {
  static_assert(N == 8 || N == 16 || N == 32, "groups of 8, 16 or 32 lanes");
  x += dpp<0xB1>(x);
  x += dpp<0x4E>(x);
  x += dpp<0x141>(x);
  if constexpr (N >= 16) x += dpp<0x140>(x);
  if constexpr (N == 32) {
    const unsigned u = __float_as_uint(x);
    const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    x = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  }
  return x;
}

// max of two floats as one v_max_f32: fmaxf on values from a lane swap makes the compiler quiet
// both inputs first (two more v_max per call, 8 per forward tile), which NaN-free scores do not
// need.
__device__ __forceinline__ float vmax(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
// max over lanes lo, lo + 16, lo + 32, lo + 48 (every lane gets it), on the VALU: the gfx950 row
// swaps pair row r of one operand with row r ^ 1 (16-lane rows), then half h with h ^ 1
// (32-lane halves); with both operands x, the max of the two results is the max of each pair.
__device__ __forceinline__ float max4_groups(float x) {
  const unsigned u = __float_as_uint(x);
  const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  x = vmax(__uint_as_float(p[0]), __uint_as_float(p[1]));
  const unsigned v = __float_as_uint(x);
  const auto q = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return vmax(__uint_as_float(q[0]), __uint_as_float(q[1]));
}

// v_permlane16_swap / v_permlane32_swap on a pair of floats (16-lane rows: the first swaps odd
// rows of a with even rows of b, the second the upper 32 lanes of a with the lower 32 of b).
__device__ __forceinline__ void swap_rows16(float& a, float& b) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false,
                                                  false);
  a = __uint_as_float(p[0]);
  b = __uint_as_float(p[1]);
}
__device__ __forceinline__ void swap_rows32(float& a, float& b) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false,
                                                  false);
  a = __uint_as_float(p[0]);
  b = __uint_as_float(p[1]);
}
// 4 x 4 transpose of float4 blocks across the lane groups g: afterwards x[j] of lane (lo, g) is
// what x[g] of lane (lo, j) was.
__device__ __forceinline__ void transpose_groups(f4& x0, f4& x1, f4& x2, f4& x3) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float a = x0[e], b = x1[e], c = x2[e], d = x3[e];
    swap_rows16(a, b);
    swap_rows16(c, d);
    swap_rows32(a, c);
    swap_rows32(b, d);
    x0[e] = a;
    x1[e] = b;
    x2[e] = c;
    x3[e] = d;
  }
}
// The contraction order of the products over head_dim: step t (of D / 4) takes from lane group g
// the dim quarter_dim(g, t / 4) + t % 4, so each MFMA adds four products, one per group:
//   D 32: 8 g + t;  D 64: 16 g + t;  D 128: 16 g + t for t < 16, 64 + 16 g + (t - 16) after
// (D 128 runs D 64's order over each half of the row). Lane (lo, g) reads float4 u of its share of
// an LDS row at dim quarter_dim(g, u). With 32 g + t at D 128, dK came out 1.7-2.5 x less accurate
// than the fp32 composed path on the reference tests' closed-form inputs (dP = dO V^T cancels
// against D there, and that order accumulated it less accurately); by halves it is 0.6-1.0 x, as
// at D 64, and no worse on N(0, 1) inputs.
template <int D>
__device__ __forceinline__ constexpr int quarter_dim(int g, int u) {
  if constexpr (D == 32) return 8 * g + 4 * u;
  return 64 * (u / 4) + 16 * g + 4 * (u % 4);
}
// The register operand of those products: dst[4 u + e] = row[quarter_dim(g, u) + e] (lane (lo, g)
// holds quarter g of its row, in the order above). At D 64 and 128 the row is read in whole
// 64-byte sectors -- load u of lane group g reads dims 16 u + 4 g .. + 3, so the four groups' loads
// of 64 dims are 64 contiguous bytes -- and a 4 x 4 transpose across the lane groups per 64 dims
// moves every float4 to its group. At D 32 each lane reads its quarter directly (two float4s).
// Two phases, so that a caller can issue other memory operations between the loads and the
// transposes (which wait for the loads): quarter_issue then quarter_place, or load_quarter for
// both. Every lane of the wave must execute them.
template <int D>
struct Quarter {
  f4 x[D == 32 ? 2 : D / 16];
};
template <int D>
__device__ __forceinline__ void quarter_issue(const float* row, int g, Quarter<D>& q) {
  if constexpr (D == 32) {
#pragma unroll
    for (int u = 0; u < 2; ++u) q.x[u] = ld4(row + 8 * g + 4 * u);
  } else {
#pragma unroll
    for (int u = 0; u < D / 16; ++u) q.x[u] = ld4(row + 16 * u + 4 * g);
  }
}
template <int D>
__device__ __forceinline__ void quarter_place(Quarter<D>& q, float (&dst)[D / 4]) {
  if constexpr (D != 32) {
    // Before: x[u] of group g holds dims 16 u + 4 g; after, x[4 i + j] holds dims
    // 64 i + 16 g + 4 j = quarter_dim(g, 4 i + j).
#pragma unroll
    for (int i = 0; i < D / 64; ++i) {
      transpose_groups(q.x[4 * i], q.x[4 * i + 1], q.x[4 * i + 2], q.x[4 * i + 3]);
    }
  }
#pragma unroll
  for (int u = 0; u < D / 16; ++u) {
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[4 * u + e] = q.x[u][e];
  }
}
template <int D>
__device__ __forceinline__ void load_quarter(const float* row, int g, float (&dst)[D / 4]) {
  Quarter<D> q;
  quarter_issue<D>(row, g, q);
  quarter_place<D>(q, dst);
}

typedef __attribute__((address_space(3))) float lds_float;
// Direct global -> LDS copy of 16 bytes per lane (global_load_lds_dwordx4): lane i's 16 bytes land
// at `lds_base` + 16 i (M0 holds the wave-uniform LDS address). Completion is counted by vmcnt,
// like a load; the caller waits (vmcnt(0)) before the barrier that precedes any read of the
// destination. Written as inline asm so that the compiler, which cannot tell which LDS buffer a
// copy targets, does not make every later LDS read wait for it (that would serialise the
// prefetch). M0 is set here and used by nothing else in these kernels. The source is a
// wave-uniform base (SGPRs) plus a per-lane byte offset below 2^32.
__device__ __forceinline__ void load_lds16(const float* base, unsigned byte_off, float* lds_base) {
  const unsigned lds = __builtin_amdgcn_readfirstlane(
      static_cast<unsigned>(reinterpret_cast<uintptr_t>((lds_float*)lds_base)));
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(byte_off), "s"(base), "s"(lds)
               : "memory");
}

// The same with the destination as an LDS byte address (wave-uniform).
__device__ __forceinline__ void load_lds16_at(const float* base, unsigned byte_off, unsigned lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(byte_off), "s"(base), "s"(lds)
               : "memory");
}
__device__ __forceinline__ void load_lds4_at(const float* base, unsigned byte_off, unsigned lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
               :
               : "v"(byte_off), "s"(base), "s"(lds)
               : "memory");
}
// The LDS byte address of an LDS object (wave-uniform).
template <typename T>
__device__ __forceinline__ unsigned lds_addr(T* p) {
  return __builtin_amdgcn_readfirstlane(
      static_cast<unsigned>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) T*)p)));
}

// The same for 4 bytes per lane (global_load_lds_dword): lane i's 4 bytes land at `lds_base` + 4 i;
// inactive lanes write nothing.
__device__ __forceinline__ void load_lds4(const float* base, unsigned byte_off, float* lds_base) {
  const unsigned lds = __builtin_amdgcn_readfirstlane(
      static_cast<unsigned>(reinterpret_cast<uintptr_t>((lds_float*)lds_base)));
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
               :
               : "v"(byte_off), "s"(base), "s"(lds)
               : "memory");
}

// s_waitcnt with vmcnt(n) and no lgkm / export wait (gfx9 encoding: vmcnt bits 3:0 and 15:14,
// expcnt 6:4, lgkmcnt 11:8). Issued through the builtin, not inline asm, so that the compiler
// knows which of its own loads have completed: otherwise it adds waits of its own at their first
// uses -- inside the loops, where they would also wait for the prefetch copies in flight. The
// empty asm keeps memory accesses from moving across the wait.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt 0..63");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
  asm volatile("" ::: "memory");
}
// Waits until every vector memory operation of this wave has completed (loads returned, stores
// and direct copies landed).
__device__ __forceinline__ void wait_mem() { wait_vm<0>(); }

// Tiles staged by direct copies are [rows][D floats], unpadded, in 16-byte chunks; chunk c of row
// r sits at position c ^ f(r). Three read patterns hit these tiles: row-wise float4 reads (lane
// (lo, g) reads row lo, chunk 4 g + u), float reads down columns (lane (lo, g): row 4 g + r,
// column 16 t + lo) and the row sums' float4 reads (16 lanes on one row, 4 rows per wave).
// On MI355X (measured with the SQ_LDS_BANK_CONFLICT counter on probe kernels): float reads are
// conflict-free when the 32 lanes of each half-wave hit 32 distinct dword banks (address mod
// 128 bytes); float4 reads follow no simple bank model, so f was chosen by measurement. For
// 256-byte rows (D 64) f is XOR-linear in the bits of r % 16 with f(1) = 3, f(2) = 9, f(4) = 12,
// f(8) = 2 (the 16 values packed in kSwz64): all three patterns conflict-free, where
// f(r) = r % 16 left the row-wise float4 reads 2-way. D 128 keeps f(r) = r % 16; D 32 (128-byte
// rows) uses f(r) = (r / 2) % 8.
constexpr unsigned long long kSwz64 = 0x47de8b1265fca930ull;
template <int D>
__device__ __forceinline__ int swz_f(int row) {
  if constexpr (D == 32) return (row >> 1) & 7;
  if constexpr (D == 64) return static_cast<int>((kSwz64 >> (4 * (row & 15))) & 15);
  return row & 15;
}
template <int D>
__device__ __forceinline__ int swz(int row, int col) {
  return row * D + ((((col >> 2) ^ swz_f<D>(row)) & (D / 4 - 1)) << 2) + (col & 3);
}

// One direct copy of 1024 bytes (16 per lane) of a [rows][D] tile: rows kCopyRows j ..
// kCopyRows (j + 1) - 1 from global (base + row * row_bytes; rows past `last` repeat row `last`)
// into the swizzled LDS tile `dst`. Lane i lands at position i % (D / 4) of row
// kCopyRows j + i / (D / 4), so it loads logical chunk (i % (D / 4)) ^ f(row).
template <int D>
constexpr int kCopyRows = 256 / D;
template <int D>
__device__ __forceinline__ void copy_part(const float* base, unsigned row_bytes, int first_row,
                                          int last_row, float* dst, int j, int lane) {
  constexpr int kC = D / 4;
  const int row = kCopyRows<D> * j + lane / kC;
  const unsigned src_row = static_cast<unsigned>(min(first_row + row, last_row));
  const unsigned c16 = 16u * static_cast<unsigned>(((lane % kC) ^ swz_f<D>(row)) & (kC - 1));
  load_lds16(base, src_row * row_bytes + c16, dst + kCopyRows<D> * j * D);
}
// The same with the tile's LDS byte address.
template <int D>
__device__ __forceinline__ void copy_part_at(const float* base, unsigned row_bytes, int first_row,
                                             int last_row, unsigned dst, int j, int lane) {
  constexpr int kC = D / 4;
  const int row = kCopyRows<D> * j + lane / kC;
  const unsigned src_row = static_cast<unsigned>(min(first_row + row, last_row));
  const unsigned c16 = 16u * static_cast<unsigned>(((lane % kC) ^ swz_f<D>(row)) & (kC - 1));
  load_lds16_at(base, src_row * row_bytes + c16, dst + 4u * kCopyRows<D> * j * D);
}

// ---------------------------------------------------------------------------------------------
// Forward. One workgroup = 4 waves x kFwdWaveQ queries of one (b, h) (QB in all); wave w owns
// queries q0 + kFwdWaveQ w .., in kFwdNT column tiles of 16 (one query per lane column lo each).
// Key tiles of KT keys are staged in LDS by direct copies (double buffered: the next tile's
// copies in flight during this tile's math) and shared by the four waves. The shapes per head_dim
// and mask are in FwdCfg below (measured on MI355X for D 64: non-causal QB 128 / KT 32, each
// K / V operand read from LDS serving two query tiles; causal QB 64 / KT 32, smaller blocks
// balancing the triangular work: at b 64 h 6 s 240 causal 42.3 us against 44.1 for KT 48, 42.1 for
// KT 16, 49.6 for QB 128 / KT 32; at b 8 h 12 s 2048 417.0 against 422.4, 421.0 and 438.5).
//   S^T = K Q^T per 16-key subtile and column tile n, D / 4 steps (the order of quarter_dim):
//   A = K[key 16 mt + lo][that dim] (LDS, float4 reads, shared by the column tiles),
//   B = Q[query lo][that dim] (registers, loaded once). Output: lane (lo, g) holds
//   S[query lo][key 16 mt + 4 g + r].
//   O^T += V^T P^T: M = dims (D / 16 tiles of 16), N = queries, contraction over the tile's keys;
//   step (kt, r) uses key 16 kt + 4 g + r, i.e. exactly the P value lane (lo, g) holds in its
//   register (kt, r). A = V[key][dim 16 mt + lo] (LDS, shared by the column tiles).
// Online softmax per query, in the log2 domain on raw scores: p = 2^(s c2 - m c2), c2 = |scale|
// log2 e (q negated for a negative scale), one fma and one exp per score. m is a reference max
// (identical in the four lanes of the query) that moves only when a tile's max exceeds it by more
// than 2^kRescaleLog2, O and the row sum being rescaled then (lazily: most tiles skip it); the row
// sum is a partial sum over the lane's own keys, combined across the four lanes once, in a fixed
// order, at the end. L = m |scale| + ln(sum).
// ---------------------------------------------------------------------------------------------

// Wave priority from the work left: 3 while more than three quarters of the walk remain, down to
// 0 for the last quarter. A SIMD otherwise issues from its oldest wave first, so the first of a
// CU's workgroups finishes well before the last, which then runs alone; with the priority falling
// as a wave progresses, co-resident waves progress together and end together.
__device__ __forceinline__ void prio_by_remaining(int rem, int total) {
  const int q = (4 * rem) / max(total, 1);
  if (q >= 3) {
    __builtin_amdgcn_s_setprio(3);
  } else if (q == 2) {
    __builtin_amdgcn_s_setprio(2);
  } else if (q == 1) {
    __builtin_amdgcn_s_setprio(1);
  } else {
    __builtin_amdgcn_s_setprio(0);
  }
}

struct FwdArgs {
  View q, k, v;
  float* o;
  float* lse;
  int B, H, S, nqb;
  float scale;
  int causal;
};

template <int D, int QB, int KT, int WAVES, bool kCausal>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(WAVES)))
fwd_kernel(FwdArgs a) {
  a.causal = kCausal ? 1 : 0;  // compile-time mask (the host launches the matching instantiation)
  constexpr int kFwdQueries = QB;          // queries per workgroup
  constexpr int kFwdWaveQ = QB / 4;        // queries per wave
  constexpr int kFwdNT = kFwdWaveQ / 16;   // 16-query column tiles per wave
  constexpr int kFwdKeys = KT;             // keys per LDS tile
  constexpr int kFwdSub = KT / 16;         // 16-key subtiles per tile
  constexpr int kQR = D / 4;               // Q values per lane and column tile
  constexpr int kDT = D / 16;              // 16-dim tiles of O
  constexpr int kCopies = KT / kCopyRows<D>;  // direct copies per K (or V) tile
  static_assert(KT % kCopyRows<D> == 0, "whole copies per tile");
  // One LDS array (each tile a constant offset from one base, folded into the LDS instructions).
  struct Smem {
    float k[2][kFwdKeys * D], v[2][kFwdKeys * D];
  };
  __shared__ __attribute__((aligned(16))) Smem sm;
  auto& sK = sm.k;
  auto& sV = sm.v;
  const unsigned lds0 = lds_addr(&sm);

  const int tid = threadIdx.x, lane = tid & 63, lo = lane & 15, g = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in an SGPR
  const int S = a.S, BH = a.B * a.H;
  int qb, bh;
  if (a.causal) {
    // Causal blocks get cheaper with the query index: the most expensive go first.
    qb = a.nqb - 1 - static_cast<int>(blockIdx.x) / BH;
    bh = static_cast<int>(blockIdx.x) % BH;
  } else {
    const int id = xcd_remap(static_cast<int>(blockIdx.x), a.nqb * BH);
    qb = id % a.nqb;
    bh = id / a.nqb;
  }
  const int b = bh / a.H, h = bh % a.H;
  const int q0 = qb * kFwdQueries;
  const int qw0 = q0 + w * kFwdWaveQ;  // the wave's first query
  const float* qp = a.q.p + b * a.q.sb + h * a.q.sh;
  const float* kp = a.k.p + b * a.k.sb + h * a.k.sh;
  const float* vp = a.v.p + b * a.v.sb + h * a.v.sh;
  // Row strides in bytes (the host guarantees every offset within a (b, h) slice < 2^32).
  const unsigned k_ss4 = static_cast<unsigned>(a.k.ss) * 4u;
  const unsigned v_ss4 = static_cast<unsigned>(a.v.ss) * 4u;

  // B operands of S^T: quarter g of Q[qi(n)] (quarter_place's order) for this lane's query in
  // column tile n, negated for a negative scale (so that the raw scores' max is the scaled
  // scores' max).
  const float qsign = a.scale < 0.0f ? -1.0f : 1.0f;
  float qr[kFwdNT][kQR];
  Quarter<D> qload[kFwdNT];  // placed into qr after the first key tile's copies are issued
#pragma unroll
  for (int n = 0; n < kFwdNT; ++n) {
    quarter_issue<D>(qp + min(qw0 + 16 * n + lo, S - 1) * a.q.ss, g, qload[n]);
  }

  // Scores enter the exponent as s * c2 (c2 = |scale| log2 e); m holds raw-score maxima.
  const float ascale = fabsf(a.scale), c2 = ascale * kLog2e;

  // Keys the block needs, and keys this wave's rows can see.
  const int k_end = a.causal ? min(S, q0 + kFwdQueries) : S;
  const int ntiles = (k_end + kFwdKeys - 1) / kFwdKeys;
  const int kw_end = a.causal ? min(S, qw0 + kFwdWaveQ) : S;
  const bool wave_live = qw0 < S;

  // Staging: wave w issues copies w, w + 4, ... of the K and V tiles; keys past S repeat key
  // S - 1 (finite; their scores are masked, so 0 * V stays 0).
  auto stage = [&](int kt0, auto bufc) {
    constexpr int buf = decltype(bufc)::value;
#pragma unroll
    for (int j0 = 0; j0 < kCopies; j0 += 4) {
      if (j0 + w < kCopies) {
        copy_part_at<D>(kp, k_ss4, kt0, S - 1, lds0 + offsetof(Smem, k[buf]), j0 + w, lane);
        copy_part_at<D>(vp, v_ss4, kt0, S - 1, lds0 + offsetof(Smem, v[buf]), j0 + w, lane);
      }
    }
  };

  f4 acc[kFwdNT][kDT];
  float m[kFwdNT], lsum[kFwdNT];
#pragma unroll
  for (int n = 0; n < kFwdNT; ++n) {
    m[n] = kNegInf;
    lsum[n] = 0.0f;
#pragma unroll
    for (int mt = 0; mt < kDT; ++mt) acc[n][mt] = zero4();
  }

  stage(0, Const<0>{});
  // Negated for a negative scale, zero past S (wave-uniform test: most waves need neither).
  const bool q_fix = a.scale < 0.0f || qw0 + kFwdWaveQ > S;
#pragma unroll
  for (int n = 0; n < kFwdNT; ++n) {
    const int qi = qw0 + 16 * n + lo;
    quarter_place<D>(qload[n], qr[n]);
    if (q_fix) {
#pragma unroll
      for (int t = 0; t < kQR; ++t) qr[n][t] = qi < S ? qr[n][t] * qsign : 0.0f;
    }
  }
  wait_mem();
  __syncthreads();
  // One key tile; unrolled by two so that the LDS buffer (t % 2) is a compile-time constant and
  // LDS addresses fold its offset into the instruction. kFull: an interior tile of the wave
  // (every key below S and, causal, none after the wave's first query) -- no liveness test, no
  // mask; the masked variant serves the rest.
  auto tile_step = [&](auto bufc, auto fullc, auto colsc, int t) {
    constexpr int buf = decltype(bufc)::value;
    constexpr bool kFull = decltype(fullc)::value != 0;
    constexpr int kCols = decltype(colsc)::value;  // column tiles with a query below S
    const int kt0 = t * kFwdKeys;
    // The next tile into the other buffer, whose last readers passed the last barrier.
    if (t + 1 < ntiles) stage(kt0 + kFwdKeys, Const<buf ^ 1>{});
    if (kFull || wave_live) {
      const float* Kt = sK[buf];
      const float* Vt = sV[buf];
      bool live[kFwdSub];
#pragma unroll
      for (int mt = 0; mt < kFwdSub; ++mt) {
        live[mt] = kFull || kt0 + 16 * mt < kw_end;  // wave-uniform
      }
      f4 s[kFwdNT][kFwdSub];
#pragma unroll
      for (int mt = 0; mt < kFwdSub; ++mt) {
#pragma unroll
        for (int n = 0; n < kFwdNT; ++n) s[n][mt] = zero4();
        if (live[mt]) {
#pragma unroll
          for (int u = 0; u < kQR / 4; ++u) {
            const f4 kk = ld4(Kt + swz<D>(16 * mt + lo, quarter_dim<D>(g, u)));
#pragma unroll
            for (int n = 0; n < kCols; ++n) {
              s[n][mt] = mma(kk.x, qr[n][4 * u], s[n][mt]);
              s[n][mt] = mma(kk.y, qr[n][4 * u + 1], s[n][mt]);
              s[n][mt] = mma(kk.z, qr[n][4 * u + 2], s[n][mt]);
              s[n][mt] = mma(kk.w, qr[n][4 * u + 3], s[n][mt]);
            }
          }
        }
      }
#pragma unroll
      for (int n = 0; n < kCols; ++n) {
        const int qi = qw0 + 16 * n + lo;
        // Mask (keys past S; causal keys after the query) and the tile's row max of the raw
        // scores (interior tiles: no mask).
        float tmax = kNegInf;
        if (kFull) {
#pragma unroll
          for (int mt = 0; mt < kFwdSub; ++mt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, s[n][mt][r]);
          }
        } else {
#pragma unroll
          for (int mt = 0; mt < kFwdSub; ++mt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int key = kt0 + 16 * mt + 4 * g + r;
              const bool ok = live[mt] && key < S && !(a.causal && key > qi);
              const float x = ok ? s[n][mt][r] : kNegInf;
              s[n][mt][r] = x;
              tmax = fmaxf(tmax, x);
            }
          }
        }
        tmax = max4_groups(tmax);
        // The row's reference max m moves only when this tile's max exceeds it by more than
        // kRescaleLog2 in the exponent (so p <= 2^kRescaleLog2); O and the row sum are rescaled
        // only when some lane's m moved (wave-uniform). A row with every key so far masked keeps
        // m = -inf.
        const bool grow = (m[n] == kNegInf && tmax != kNegInf) || (tmax - m[n]) * c2 > kRescaleLog2;
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
          // (From m = -inf: nothing accumulated yet, alpha 0, also when c2 = 0.)
          const float alpha = !grow ? 1.0f : m[n] == kNegInf ? 0.0f : exp2_hw((m[n] - tmax) * c2);
          if (grow) m[n] = tmax;
          lsum[n] *= alpha;
#pragma unroll
          for (int mt = 0; mt < kDT; ++mt) acc[n][mt] *= alpha;
        }
        // p = 2^(s c2 - m c2): one fma per score.
        const float mc = m[n] * c2;
        float psum = 0.0f;
        if (kFull) {
#pragma unroll
          for (int mt = 0; mt < kFwdSub; ++mt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float p = exp2_hw(fmaf(s[n][mt][r], c2, -mc));
              s[n][mt][r] = p;
              psum = mt == 0 && r == 0 ? p : psum + p;
            }
          }
        } else {
          // Masked scores are -inf: select 0 for them (the fma would give NaN for -inf * 0 or
          // -inf + inf).
#pragma unroll
          for (int mt = 0; mt < kFwdSub; ++mt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float x = s[n][mt][r];
              const float p = x == kNegInf ? 0.0f : exp2_hw(fmaf(x, c2, -mc));
              s[n][mt][r] = p;
              psum = mt == 0 && r == 0 ? p : psum + p;
            }
          }
        }
        lsum[n] += psum;
      }
#pragma unroll
      for (int kt = 0; kt < kFwdSub; ++kt) {
        if (!live[kt]) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
          for (int mt = 0; mt < kDT; ++mt) {
            const float vv = Vt[swz<D>(16 * kt + 4 * g + r, 16 * mt + lo)];
#pragma unroll
            for (int n = 0; n < kCols; ++n) acc[n][mt] = mma(vv, s[n][kt][r], acc[n][mt]);
          }
        }
      }
    }
    wait_mem();       // the next tile's copies have landed
    __syncthreads();  // and every wave is done with this tile's buffers
  };
  // Interior tiles of this wave: tiles whose keys are all below S and, causal, all at or before
  // the wave's first query (wave-uniform); none for a wave whose queries run past S. A wave with
  // its last column tile wholly past S (two column tiles, the second dead) computes only the
  // first.
  const bool all_cols = qw0 + kFwdWaveQ - 16 < S;
  const int full_end =
      qw0 + kFwdWaveQ <= S ? (a.causal ? min(S, qw0 + 1) : S) / kFwdKeys : 0;
  auto step = [&](auto bufc, int t) {
    if (wave_live && t < full_end) {
      tile_step(bufc, Const<1>{}, Const<kFwdNT>{}, t);
    } else if (kFwdNT != 2 || all_cols) {
      tile_step(bufc, Const<0>{}, Const<kFwdNT>{}, t);
    } else {
      tile_step(bufc, Const<0>{}, Const<1>{}, t);
    }
  };
  // Non-causal only (every workgroup walks all tiles): at config 2 the forward is 4 % faster. The
  // causal walks differ in length, and the same rule was 0.6-2 % slower there; step 2 was 5 %
  // slower with it (its waves hide each other's stalls best out of phase).
  for (int t = 0; t < ntiles; t += 2) {
    if (!a.causal) prio_by_remaining(ntiles - t, ntiles);
    step(Const<0>{}, t);
    if (t + 1 < ntiles) step(Const<1>{}, t + 1);
  }

  if (wave_live) {
    float lrow[kFwdNT];  // L of this lane's row in each column tile
#pragma unroll
    for (int n = 0; n < kFwdNT; ++n) {
      // The row sum: the four lanes of a query hold partial sums over disjoint keys; every lane
      // adds them in the same order.
      const float l0 = __shfl(lsum[n], lo), l1 = __shfl(lsum[n], lo + 16);
      const float l2 = __shfl(lsum[n], lo + 32), l3 = __shfl(lsum[n], lo + 48);
      const float l = (l0 + l1) + (l2 + l3);
      lrow[n] = m[n] * ascale + logf(l);
      // O as whole 128-byte lines per store instruction (row-wise 64-byte pieces reached HBM
      // unmerged: 33.5 MB written at b 64 h 6 s 240 for 24.0 MB of O and L; 24.0 MB this way).
      // Lane (lo, g) holds dims 16 mt + 4 g .. + 3 of row lo; for each pair of dim tiles
      // (2 p, 2 p + 1) lanes lo and lo ^ 8 swap a float4 (DPP row rotate by 8), so that the first
      // store writes rows 0-7 and the second rows 8-15 of the column tile, each row's dims
      // 32 p .. 32 p + 31 whole: lanes lo < 8 the first 16 of them, lanes lo >= 8 the second 16.
      // Rows past S hold garbage and are not stored.
      const float inv = 1.0f / l;
      const bool hi = lo >= 8;
      const int r1 = qw0 + 16 * n + (lo & 7), r2 = r1 + 8;
      float* const o1 = a.o + ((static_cast<int64_t>(b) * S + r1) * a.H + h) * D;
      float* const o2 = o1 + static_cast<int64_t>(8) * a.H * D;
#pragma unroll
      for (int p = 0; p < kDT / 2; ++p) {
        const f4 A = acc[n][2 * p] * inv, B = acc[n][2 * p + 1] * inv;
        f4 R;
#pragma unroll
        for (int e = 0; e < 4; ++e) R[e] = dpp<0x128>(hi ? A[e] : B[e]);
        const int col = 32 * p + (hi ? 16 : 0) + 4 * g;
        if (r1 < S) st4_nt(o1 + col, hi ? R : A);
        if (r2 < S) st4_nt(o2 + col, hi ? B : R);
      }
    }
    // L of column tile g from lane group g: one store covers the wave's rows.
    if (g < kFwdNT) {
      const int qi = qw0 + 16 * g + lo;
      const float lv = kFwdNT == 2 && g == 1 ? lrow[kFwdNT - 1] : lrow[0];
      if (qi < S) __builtin_nontemporal_store(lv, a.lse + static_cast<int64_t>(bh) * S + qi);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Backward, step 1: D[b, h, i] = sum_c dO[b, i, h, c] O[b, i, h, c]. D / 4 lanes per row (one
// float4 each, then lane_sum: one fixed order). It also clears the turn counters, the ticket and
// the guard word of step 2 (stream order puts it first).
// ---------------------------------------------------------------------------------------------
template <int D>
__global__ void __launch_bounds__(kThreads) prep_kernel(const float* __restrict__ o, View d_o,
                                                       float* __restrict__ dsum,
                                                       int* __restrict__ turn,
                                                       int* __restrict__ ctrl, int B, int H,
                                                       int S, int nturn) {
  constexpr int kLanes = D / 4;  // lanes per row
  // 64-bit: the grid holds up to b h s / (kThreads / kLanes) workgroups of kThreads threads.
  const int64_t gtid = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (gtid < nturn) turn[gtid] = 0;
  if (gtid < 64) ctrl[gtid] = 0;
  const int64_t rows = static_cast<int64_t>(B) * H * S;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (kThreads / kLanes) + (threadIdx.x / kLanes);
  const int c4 = threadIdx.x % kLanes;
  float x = 0.0f;
  if (row < rows) {
    const int i = static_cast<int>(row % S);
    const int64_t bh = row / S;
    const int h = static_cast<int>(bh % H), b = static_cast<int>(bh / H);
    const f4 ov = ld4(o + ((static_cast<int64_t>(b) * S + i) * H + h) * D + 4 * c4);
    const f4 gv = ld4(d_o.p + b * d_o.sb + h * d_o.sh + i * d_o.ss + 4 * c4);
    x = ov.x * gv.x;
    x = fmaf(ov.y, gv.y, x);
    x = fmaf(ov.z, gv.z, x);
    x = fmaf(ov.w, gv.w, x);
  }
  x = lane_sum<kLanes>(x);
  if (row < rows && c4 == 0) dsum[row] = x;
}

// ---------------------------------------------------------------------------------------------
// Backward, step 2. One workgroup = one key block of 64 keys of one (b, h) (split: by workgroup
// index; turns: by ticket); wave w owns keys k0 + 16 w .. + 15, one per lane column lo, with K and
// V of its key in registers (the B operands of S and dP), the block's K in the layout of the dQ
// product's B operand (registers too), and dK^T, dV^T of its keys in accumulators. It walks query
// tiles of kQT = 16 (kNS = 1 subtile m of 16 queries; causal: from the block's first key on), the
// next tile's Q, dO, L, D in flight during this one (LDS double buffer, filled by direct global ->
// LDS copies).
//   S = Q K^T and dP = dO V^T per subtile: M = queries, N = the wave's keys, contraction over the
//   D dims in D / 4 steps (the order of quarter_dim): A = Q / dO [query 16 m + lo][that dim]
//   (LDS, float4 reads), B = K / V [key lo][that dim].
//   P = exp(S scale - L), dS = P o (dP - D), in place in the accumulators.
//   dV^T += dO^T P, dK^T += Q^T dS: M = dims (D / 16 tiles), N = keys, contraction over the tile's
//   queries; step (m, r) uses query 16 m + 4 g + r: the P / dS value lane (lo, g) holds in register
//   r of subtile m.
//   dQ partial = dS K over the block's 64 keys: dS goes through LDS (the one product that needs
//   queries in lo); wave w computes the 16-dim tiles dt = w, w + 4, ... (< D / 16; at D 32 waves 2
//   and 3 have none), step t contracting keys 16 g + t: A = dS[16 m + lo][16 g + t] (LDS, float4
//   reads), B = K[k0 + 16 g + t][16 dt + lo] (registers).
// split: the partial is stored to the key block's slot at the start of the next tile (plain
// stores, nothing waits for them); step 3 (dq_kernel) sums the slots.
// turns: the partial is added into dQ on the tile's turn, one tile later (software pipelined:
// while tile t + 1's products run, the loads of what the earlier key blocks summed for tile t are
// in flight): the first contributor stores, the others add their partial to what they read, the
// last contributor scales; then the turn passes to the next key block.
// Either way a tile's dQ is ((p_0 + p_1) + p_2) + ... in a fixed key-block order, times scale.
// ---------------------------------------------------------------------------------------------
#ifndef BWD_WAVES
#define BWD_WAVES 3
#endif
constexpr int kQT = kBwdQueryTile;
constexpr int kOwnDMaxBlocks = 4;  // D 128 split: step 2 forms D up to this many key blocks
constexpr int kNS = kQT / 16;  // 16-query subtiles per tile
constexpr int kBwdLd = 68;     // pitch (floats) of the transposed K tile at D 128
// Q and dO tiles are [kQT rows][D floats] in the swizzled layout of swz(), filled by direct copies.

struct BwdArgs {
  View q, k, v, d_o;
  const float* o;     // split, D <= 64: the forward's output [b, s, h, D] (D = rowsum(dO o O)
                      // computed here)
  const float* lse;
  const float* dsum;  // otherwise: D from step 1
  float* dqkv;
  float* part;  // split: the dQ partials, [nkb][b h][ntile][kQT * D] in fragment order
  // split, D <= 64, null when step 3 sums every tile: per key block, the epoch of the launch
  // that finished it or'ed with its XCD; per query tile, the epoch of the launch that summed it
  // here; the workspace's record of this launch's epoch. Workgroups from n_main on sum tiles;
  // n_main (the key blocks, rounded up to a multiple of 8) and the sums' plan (sum_plan, the same
  // one the host sized the grid with).
  unsigned long long* arrive;
  unsigned long long* done;
  unsigned long long* epoch_slot;
  unsigned long long epoch;
  int n_main;
  SumPlan plan;
  int* turn;
  int* ctrl;
  int B, H, S, nkb, ntile;
  float scale;
  int causal;
  int stagger;  // non-causal only: spread the key blocks' walks over the tiles (see below)
  int kkeys;    // keys per key block (split: 64 KG)
  // The (b, h) this launch covers: bh0 .. bh0 + nbh - 1 (the split path may run the (b, h) in
  // chunks, each with its partials, arrival slots and done flags at the start of the workspace;
  // the turn path always covers all, bh0 0 and nbh b h).
  int bh0, nbh;
  // 1: no step 3 follows (step 2's sums cover every tile): a sum's wait is bounded only by
  // kSumPollsFinal and one that gives up raises the guard word and leaves NaN in its rows.
  int sums_final;
  // Test hook (0 in use): the non-causal summing workgroups of XCD x take the (b, h)s of XCD
  // x + sum_shift, so that every sum reads partials written on another XCD.
  int sum_shift;
  // Test hook (-1 in use): the dQ sums of this (b, h) (its index in the whole backward) give up
  // before their first poll, as a wait that timed out would.
  int give_up_bh;
};

// Staggered walks make a key block wait on blocks of its own (b, h) that hold later tickets; that
// cannot deadlock while all key blocks of one (b, h) can be resident at once, which holds for up
// to this many per (b, h) on any MI355X partition. Longer sequences use the index order.
constexpr int kStaggerMaxBlocks = 64;

// The dQ hand-over between key blocks. MI355X has one L2 per XCD and the L2s are not coherent
// with each other, so an agent-scope release / acquire fence pair has to write back / invalidate
// a whole L2 -- per tile, per workgroup, far more than the 32 x 64 floats that change hands. The
// hand-over therefore uses accesses that are coherent at agent scope one by one instead: the
// turn counter and the dQ values are read and written with relaxed agent-scope atomics
// (global loads / stores with the sc1 scope bit: served at the agent coherence point, not from a
// stale L2 line), and the writer waits for its dQ stores to complete (vmcnt(0)) before the turn
// store is issued (after a workgroup barrier, so every wave's stores are complete). A reader
// issues its dQ loads only after it has seen the turn, so it reads the completed values.
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() { wait_mem(); }
__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }
// Vector memory operations complete in issue order (vmcnt counts them down in order), so
// wait_vm<n> waits for everything but the last n operations issued: stage 1's loads (turns) or the
// partial's stores (split), the last operations before a tile's first barrier.

// Spin until the turn counter reads `want`. Bounded: on timeout the guard word is raised and
// the wait returns false (the turn never came: what the earlier key blocks summed is incomplete).
__device__ __forceinline__ bool wait_turn(int* p, int want, int* guard) {
  int spins = 0;
  while (__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != want) {
    __builtin_amdgcn_s_sleep(2);
    ++spins;
    // Once any wait of this launch has timed out, the others stop waiting too.
    if (spins > kSpinBound ||
        ((spins & 63) == 0 &&
         __hip_atomic_load(guard, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0)) {
      __hip_atomic_store(guard, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
  }
  return true;
}

// Occupancy target: BWD_WAVES waves per SIMD (the kernel is latency-bound: with fewer, the
// matrix cores idle behind barriers), 2 at D 128 (its registers do not fit 3).
template <int D>
__device__ __forceinline__ void bwd_sum_tiles(const BwdArgs& a, int x, int m, unsigned* flag);
template <int D, int NT>
__device__ __forceinline__ void bwd_sum_range(const BwdArgs& a, int bh, int j0, int j1,
                                              unsigned* flag);

// kOwnSums (split, causal): each key block sums the dQ tiles it completes after its walk; a
// separate instantiation, so that the non-causal kernel's registers are not spent on it.
template <bool kSplit, int D, bool kOwnSums = false, bool kOwnD = false>
__global__ void __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(D == 128 ? 2 : BWD_WAVES))) bwd_kernel(BwdArgs a) {
  constexpr int kKR = D / 4;                  // K (or V) values per lane: B operands of S, dP
  constexpr int kDT = D / 16;                 // 16-dim tiles (dK, dV accumulators; dQ tiles)
  constexpr int kDQ = (kDT + 3) / 4;          // dQ tiles per wave (w, w + 4, ...)
  constexpr int kCopies = kQT / kCopyRows<D>;  // direct copies per Q (or dO) tile
  // D 128: the dQ product's K comes from LDS (transposed, [D][kBwdLd]), its registers would not
  // fit beside the others.
  constexpr bool kKtLds = D == 128;
  __shared__ __attribute__((aligned(16))) float sKt[kKtLds ? D * kBwdLd : 4];
  static_assert(!kSplit || D == 128, "the split mode at D <= 64 is bwd_split_kernel");
  // D = rowsum(dO o O): from step 1, or (kOwnD, split only: few key blocks per (b, h)) formed
  // here from O rows staged beside dO in one buffer (the two workgroups a CU holds have LDS for
  // one, not two).
  static_assert(!kOwnD || kSplit, "D is formed in step 2 in the split mode only");
  // The split instantiations know the mask (kOwnSums is the causal one): every test folds away.
  if constexpr (kSplit) a.causal = kOwnSums ? 1 : 0;
  __shared__ __attribute__((aligned(16))) float sQ[2][kQT * D];
  __shared__ __attribute__((aligned(16))) float sdO[2][kQT * D];
  // dS [kQT][64 keys], swizzled like a D 64 tile (its writes are column reads' pattern, its
  // reads row-wise float4 reads).
  __shared__ __attribute__((aligned(16))) float sdS[kQT * kBwdKeys];
  __shared__ __attribute__((aligned(16))) float sL[2][kQT];
  __shared__ __attribute__((aligned(16))) float sD[2][kQT];
  __shared__ __attribute__((aligned(16))) float sO[kOwnD ? kQT * D : 4];
  __shared__ int s_item;
  __shared__ unsigned s_flag;  // a dQ sum's poll result (split)

  const int tid = threadIdx.x, lane = tid & 63, lo = lane & 15, g = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in an SGPR
  const int BH = a.B * a.H;
  int item;
  if (kSplit) {
    // No workgroup waits on another: the workgroup index is the item. Non-causal: the key blocks
    // of one (b, h) on one XCD (they read the same Q and dO tiles at about the same time), and
    // the dQ sums of step 2's tail in the workgroups appended to the grid (as bwd_split_kernel's).
    // Causal: round-robin over the XCDs, which spreads the expensive low blocks evenly.
    const int n = a.nkb * BH, id = static_cast<int>(blockIdx.x);
    if (a.arrive != nullptr && id == 0 && tid == 0) *a.epoch_slot = a.epoch;  // for step 3
    if (a.arrive != nullptr && id >= n) {
      if (id >= a.n_main) bwd_sum_tiles<D>(a, id & 7, (id - a.n_main) >> 3, &s_flag);
      return;
    }
    item = a.causal ? id : xcd_remap(id, n);
    // No turn waits here: the guard word reads 0 (unless a final sum's wait gave up; written
    // through, as that raise is, so that no copy of it lingers in this XCD's L2).
    if (id == 0 && tid == 0) {
      __hip_atomic_store(a.ctrl + kCtrlGuard, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  } else {
    // Ticket: the key block this workgroup computes, in arrival order. Key block kb of a (b, h)
    // has a later item than kb - 1, so the block it waits on was taken by an earlier, running
    // workgroup.
    if (tid == 0) s_item = atomicAdd(a.ctrl + kCtrlTicket, 1);
    __syncthreads();
    item = s_item;
    if (item >= a.nkb * BH) {
      // The ticket was not cleared by step 1 on this workspace: refuse (no access out of range),
      // and raise the guard word so the caller can tell.
      if (tid == 0) {
        __hip_atomic_store(a.ctrl + kCtrlGuard, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      return;
    }
  }
  // Non-causal: (b, h)-major, the key blocks of one (b, h) adjacent. Causal: key-block-major, so
  // the expensive low blocks (they see every later query) start first. Either way key block kb
  // of a (b, h) comes after kb - 1.
  const int bh = a.causal ? item % BH : item / a.nkb;
  const int kb = a.causal ? item / BH : item % a.nkb;
  const int b = bh / a.H, h = bh % a.H, S = a.S;
  const int k0 = kb * kBwdKeys;
  const int kw0 = k0 + 16 * w;  // the wave's first key
  const int key = kw0 + lo;     // this lane's key
  const bool wave_dq = w < kDT;  // the wave computes dQ tiles (all waves but 2, 3 at D 32)
  int* const guard = a.ctrl + kCtrlGuard;

  const float* qp = a.q.p + b * a.q.sb + h * a.q.sh;
  const float* kp = a.k.p + b * a.k.sb + h * a.k.sh;
  const float* vp = a.v.p + b * a.v.sb + h * a.v.sh;
  const float* gp = a.d_o.p + b * a.d_o.sb + h * a.d_o.sh;
  const float* lp = a.lse + static_cast<int64_t>(bh) * S;
  const float* dp = a.dsum + static_cast<int64_t>(bh) * S;
  int* tp = a.turn + static_cast<int64_t>(bh) * a.ntile;
  // Row strides in bytes (the host guarantees every offset within a (b, h) slice < 2^32).
  const unsigned q_ss4 = static_cast<unsigned>(a.q.ss) * 4u;
  const unsigned g_ss4 = static_cast<unsigned>(a.d_o.ss) * 4u;
  // dQ of query qi, dim tile dt: element 16 dt + lo + qi * dq_row of dq_base (part 0 of the
  // [b, s, 3, h, D] gradient); the host guarantees s * 3 h * D < 2^32.
  float* const dq_base = a.dqkv + static_cast<int64_t>(b) * S * 3 * a.H * D +
                         static_cast<int64_t>(h) * D;
  const unsigned dq_row = 3u * static_cast<unsigned>(a.H) * D;

  // B operands of S and dP: quarter g of K[key] (quarter_place's order), V likewise; of the dQ
  // product: kQ[j][t] = K[k0 + 16 g + t][16 (w + 4 j) + lo]. Zero past S.
  float kB[kKR], vB[kKR], kQ[kKtLds ? 1 : kDQ][16];
  {
    const int kr = min(key, S - 1);
    load_quarter<D>(kp + kr * a.k.ss, g, kB);
    load_quarter<D>(vp + kr * a.v.ss, g, vB);
#pragma unroll
    for (int t = 0; t < kKR; ++t) {
      kB[t] = key < S ? kB[t] : 0.0f;
      vB[t] = key < S ? vB[t] : 0.0f;
    }
  }
  if constexpr (kKtLds) {
    // sKt[dim][key] = K[k0 + key][dim] (zero past S); read after the first barrier below.
    for (int i = tid; i < kBwdKeys * (D / 4); i += kThreads) {
      const int kl = i / (D / 4), c = i % (D / 4), kk = k0 + kl;
      const f4 x = kk < S ? ld4(kp + kk * a.k.ss + 4 * c) : zero4();
#pragma unroll
      for (int e = 0; e < 4; ++e) sKt[(4 * c + e) * kBwdLd + kl] = x[e];
    }
  } else {
#pragma unroll
    for (int j = 0; j < kDQ; ++j) {
      const int dt = w + 4 * j;
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const int kk = k0 + 16 * g + t;
        kQ[j][t] = kk < S && dt < kDT ? kp[kk * a.k.ss + 16 * dt + lo] : 0.0f;
      }
    }
  }

  // Staging of one query tile, all by direct copies (nothing passes through registers, so no
  // wait is needed before the barrier that precedes the tile): wave w issues copies w, w + 4, ...
  // of the Q and dO tiles (copy_part), and of the O tile where D is formed here; wave 0 copies
  // the tile's L, wave 1 its D from step 1 (lanes 0..kQT-1, one float each). Rows past S repeat
  // row S - 1 (finite; masked later).
  const float* const op = a.o + (static_cast<int64_t>(b) * S * a.H + h) * D;
  const unsigned o_ss4 = static_cast<unsigned>(a.H) * D * 4u;
  auto gload = [&](int q0, int buf) {
#pragma unroll
    for (int j0 = 0; j0 < kCopies; j0 += 4) {
      if (j0 + w < kCopies) {
        copy_part<D>(qp, q_ss4, q0, S - 1, sQ[buf], j0 + w, lane);
        copy_part<D>(gp, g_ss4, q0, S - 1, sdO[buf], j0 + w, lane);
        if constexpr (kOwnD) copy_part<D>(op, o_ss4, q0, S - 1, sO, j0 + w, lane);
      }
    }
    if (kOwnD ? w == 0 : w < 2) {
      if (lane < kQT) {
        const unsigned off = 4u * static_cast<unsigned>(min(q0 + lane, S - 1));
        load_lds4(w == 0 ? lp : dp, off, w == 0 ? sL[buf] : sD[buf]);
      }
    }
  };
  // D of the tile staged in buffer `buf` from its O and dO rows (as step 1: D / 4 lanes per row,
  // the same operations in the same order).
  auto form_d = [&](int buf) {
    constexpr int kLanes = D / 4;
    // The addresses are recomputed at each call (the empty asm hides that they do not change):
    // held across the walk, they pushed the kernel's registers past 256.
    int tv = tid;
    asm volatile("" : "+v"(tv));
#pragma unroll
    for (int i0 = 0; i0 < kQT * kLanes; i0 += kThreads) {
      const int i = i0 + tv, row = i / kLanes, c4 = i % kLanes;
      const f4 ov = ld4(&sO[swz<D>(row, 4 * c4)]);
      const f4 gv = ld4(&sdO[buf][swz<D>(row, 4 * c4)]);
      float x = ov.x * gv.x;
      x = fmaf(ov.y, gv.y, x);
      x = fmaf(ov.z, gv.z, x);
      x = fmaf(ov.w, gv.w, x);
      x = lane_sum<kLanes>(x);
      if (c4 == 0) sD[buf][row] = x;
    }
  };
  // The order in which key blocks add into a tile's dQ (fixed by the shape alone, so every run
  // sums in the same order), chosen so that a block's predecessor reaches the tile first:
  //   causal: blocks 0 .. last (those holding a key <= the tile's last query), in index order;
  //     block kb walks tiles upward from its first key, after the lower blocks (ticket order);
  //   non-causal: block kb walks all tiles starting at t0(kb) = kb ntile / nkb (wrapping), so the
  //     blocks are spread over the tiles; tile j's order is the order in which the blocks reach it
  //     in that walk: kb* (the last block with t0 <= j) first, then kb* - 1, ..., 0, then
  //     nkb - 1, ..., kb* + 1. Its predecessor is then about ntile / nkb tiles ahead of it.
  //     (Without `stagger`: every block walks from tile 0 and the order is 0 .. nkb - 1.)
  // pos_of: this block's position in tile j's order; count_of: the number of contributors.
  const int t0 = a.causal ? k0 / kQT : (a.stagger ? (kb * a.ntile) / a.nkb : 0);
  const int nsteps = a.causal ? a.ntile - t0 : a.ntile;
  auto tile_at = [&](int step) {
    const int j = t0 + step;
    return a.causal ? j : (j >= a.ntile ? j - a.ntile : j);
  };
  auto pos_of = [&](int j) {
    if (a.causal || !a.stagger) return kb;
    const int kstar = min(a.nkb - 1, (j * a.nkb + a.nkb - 1) / a.ntile);
    return kstar >= kb ? kstar - kb : kstar - kb + a.nkb;
  };
  auto count_of = [&](int j) {
    return a.causal ? min(a.nkb - 1, min(S - 1, j * kQT + kQT - 1) / kBwdKeys) + 1 : a.nkb;
  };

  f4 dva[kDT], dka[kDT];
#pragma unroll
  for (int mt = 0; mt < kDT; ++mt) {
    dva[mt] = zero4();
    dka[mt] = zero4();
  }
  // The dQ hand-over runs two tiles behind the products (software pipelined):
  //   stage 1 (iteration j + 1): wait for tile j's turn, load what the earlier key blocks summed
  //     -- in flight during that iteration's products;
  //   stage 2 (iteration j + 2): add this block's partial, store -- the stores complete during
  //     that iteration's products, before its first barrier, after which the turn passes.
  // p1: partial computed, sums not yet loaded; p2: sums loaded, not yet stored. For each: the
  // tile's first query (-1: none), this block's position in the tile's order, the contributors.
  int p1_q0 = -1, p1_pos = 0, p1_cnt = 1, p2_q0 = -1, p2_pos = 0, p2_cnt = 1;
  f4 p1[kDQ][kNS], p2[kDQ][kNS];
  float p1s[kDQ][kNS][4], p2s[kDQ][kNS][4];
#pragma unroll
  for (int j = 0; j < kDQ; ++j) {
#pragma unroll
    for (int m = 0; m < kNS; ++m) {
      p1[j][m] = zero4();
      p2[j][m] = zero4();
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p1s[j][m][r] = 0.0f;
        p2s[j][m][r] = 0.0f;
      }
    }
  }
  // Stage 1 for the tile at q0p (waves with dQ tiles): wait for the turn (one lane polls), then
  // load. Exactly kStage1Loads load instructions are issued (rows past S read row S - 1, unused),
  // the last vector memory operations before the iteration's first barrier, so that barrier need
  // not wait for them. A wait that gave up (the guard word is raised) makes the loaded sums NaN,
  // so the tile's dQ reads NaN instead of a silently incomplete sum.
  constexpr int kStage1Loads = 4 * kNS * kDQ;
  auto load_sums = [&](int q0p, int pos, int seen, float (&sums)[kDQ][kNS][4]) {
    if (pos == 0 || !wave_dq) return;
    int gave_up = 0;
    if (lane == 0 && seen != pos) gave_up = wait_turn(tp + q0p / kQT, pos, guard) ? 0 : 1;
    // Every lane is active here (the tests above are wave-uniform): lane 0's result for all. Or'ed
    // into the loaded bits, 0x7fc00000 makes any value a quiet NaN and 0 leaves it as it is (the
    // loads stay unconditional, so their count before the barrier does not change).
    const int poison = __builtin_amdgcn_readfirstlane(gave_up) ? 0x7fc00000 : 0;
    compiler_fence();
#pragma unroll
    for (int j = 0; j < kDQ; ++j) {
#pragma unroll
      for (int m = 0; m < kNS; ++m) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int qi = min(q0p + 16 * m + 4 * g + r, S - 1);
          const float x = ld_agent(dq_base + (16u * (w + 4 * j) + lo + qi * dq_row));
          sums[j][m][r] = __int_as_float(__float_as_int(x) | poison);
        }
      }
    }
    compiler_fence();
  };
  // Stage 2: the running sum plus this block's partial (x scale by the last contributor).
  auto store_sums = [&](int q0p, int pos, int cnt, const f4 (&part)[kDQ][kNS],
                        const float (&sums)[kDQ][kNS][4]) {
    if (!wave_dq) return;
#pragma unroll
    for (int j = 0; j < kDQ; ++j) {
#pragma unroll
      for (int m = 0; m < kNS; ++m) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int qi = q0p + 16 * m + 4 * g + r;
          if (qi < S) {
            float x = pos > 0 ? sums[j][m][r] + part[j][m][r] : part[j][m][r];
            if (pos == cnt - 1) x *= a.scale;
            st_agent(dq_base + (16u * (w + 4 * j) + lo + qi * dq_row), x);
          }
        }
      }
    }
  };
  // split: this block's partial of the tile at q0p into its slot, in fragment order (register r
  // of lane l for dim tile dt of subtile m at (m kDT + dt) 256 + 4 l + r: one contiguous 1 KB
  // store per dim tile and subtile).
  constexpr int kPartStores = kNS * kDQ;
  auto store_part = [&](int q0p, const f4 (&part)[kDQ][kNS]) {
    if (!wave_dq) return;
    const float* dst = a.part + ((static_cast<int64_t>(kb) * BH + bh) * a.ntile + q0p / kQT) *
                                    (kQT * D);
#pragma unroll
    for (int j = 0; j < kDQ; ++j) {
#pragma unroll
      for (int m = 0; m < kNS; ++m) {
        st4_dev(dev_rsrc(dst + (m * kDT + w + 4 * j) * 256, 1024), 16u * lane, part[j][m]);
      }
    }
  };
  // After stage 2's stores completed (vmcnt(0) and a barrier): the next contributor's turn.
  auto pass_turn = [&](int q0p, int pos, int cnt) {
    if (pos + 1 < cnt && tid == 0) {
      __hip_atomic_store(tp + q0p / kQT, pos + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  };

  // Causal: the walk starts at the block's first key (earlier queries see none of its keys).
  gload(tile_at(0) * kQT, 0);
  wait_stores();  // the direct copies have landed
  __syncthreads();
  if constexpr (kOwnD) {
    form_d(0);
    __syncthreads();
  }
  // One tile; `bufc()` is the LDS buffer, t % 2. The split kernel unrolls the walk by two so that
  // it is a compile-time constant there and LDS addresses fold the buffer offset into the
  // instruction (the turn kernel has no registers to spare for that).
  auto tile_step = [&](auto bufc, int t) {
    const int buf = bufc();
    const int q0 = tile_at(t) * kQT;
    const bool has_next = t + 1 < nsteps;
    // The next tile into the other buffer, whose last readers passed the last barrier.
    if (has_next) gload(tile_at(t + 1) * kQT, buf ^ 1);
    const float* Qt = sQ[buf];
    const float* Gt = sdO[buf];
    int seen = -1;
    if (kSplit) {
      if (p1_q0 >= 0) store_part(p1_q0, p1);  // the last tile's partial
    } else {
      // Stage 1's turn, read early (one lane, no wait here): by the time it is checked below the
      // value has arrived, and usually the turn with it.
      if (p1_q0 >= 0 && p1_pos > 0 && wave_dq && lane == 0) {
        seen = __hip_atomic_load(tp + p1_q0 / kQT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      if (p2_q0 >= 0) store_sums(p2_q0, p2_pos, p2_cnt, p2, p2s);  // stage 2, two tiles back
    }
    compiler_fence();

    // Wave-uniform liveness of each 16-query subtile for this wave's 16 keys.
    bool live[kNS];
#pragma unroll
    for (int m = 0; m < kNS; ++m) {
      const int qm0 = q0 + 16 * m;
      live[m] = qm0 < S && kw0 < S && !(a.causal && kw0 > qm0 + 15);
    }

    // S and dP.
    f4 sS[kNS], sP[kNS];
#pragma unroll
    for (int m = 0; m < kNS; ++m) {
      sS[m] = zero4();
      sP[m] = zero4();
      if (!live[m]) continue;
#pragma unroll
      for (int u = 0; u < kKR / 4; ++u) {
        const int at = swz<D>(16 * m + lo, quarter_dim<D>(g, u));
        const f4 x = ld4(Qt + at), y = ld4(Gt + at);
        sS[m] = mma(x.x, kB[4 * u], sS[m]);
        sS[m] = mma(x.y, kB[4 * u + 1], sS[m]);
        sS[m] = mma(x.z, kB[4 * u + 2], sS[m]);
        sS[m] = mma(x.w, kB[4 * u + 3], sS[m]);
        sP[m] = mma(y.x, vB[4 * u], sP[m]);
        sP[m] = mma(y.y, vB[4 * u + 1], sP[m]);
        sP[m] = mma(y.z, vB[4 * u + 2], sP[m]);
        sP[m] = mma(y.w, vB[4 * u + 3], sP[m]);
      }
    }

    if (!kSplit && p1_q0 >= 0) load_sums(p1_q0, p1_pos, seen, p1s);  // stage 1, one tile back

    // P = exp(S scale - L), dS = P o (dP - D); lane (lo, g), register r of subtile m: query
    // q0 + 16 m + 4 g + r, key `key`. Then dV^T and dK^T.
#pragma unroll
    for (int m = 0; m < kNS; ++m) {
      if (!live[m]) continue;
      const f4 Lv = ld4(&sL[buf][16 * m + 4 * g]), Dv = ld4(&sD[buf][16 * m + 4 * g]);
      const int qi0 = q0 + 16 * m + 4 * g;
      if ((!a.causal || kw0 + 15 <= q0 + 16 * m) && q0 + 16 * m + 16 <= S && kw0 + 16 <= S) {
        // Every query and key of the subtile is live (wave-uniform test; causal: every key at or
        // before every query): no mask.
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = exp2_hw(fmaf(sS[m][r], a.scale, -Lv[r]) * kLog2e);
          sP[m][r] = p * (sP[m][r] - Dv[r]);  // dS
          sS[m][r] = p;                        // P
        }
      } else {
        // Masked: keys past S, queries past S, causal keys after the query (the exponent is
        // finite for every staged row, and the select drops it).
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool ok = qi0 + r < S && key < S && !(a.causal && key > qi0 + r);
          const float e = exp2_hw(fmaf(sS[m][r], a.scale, -Lv[r]) * kLog2e);
          const float p = ok ? e : 0.0f;
          sP[m][r] = p * (sP[m][r] - Dv[r]);  // dS
          sS[m][r] = p;                        // P
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
#pragma unroll
        for (int mt = 0; mt < kDT; ++mt) {
          const int at = swz<D>(16 * m + 4 * g + r, 16 * mt + lo);
          dva[mt] = mma(Gt[at], sS[m][r], dva[mt]);
          dka[mt] = mma(Qt[at], sP[m][r], dka[mt]);
        }
      }
    }

    // This tile's dS into LDS (zero where the wave's keys are all masked).
#pragma unroll
    for (int m = 0; m < kNS; ++m) {
#pragma unroll
      for (int r = 0; r < 4; ++r) sdS[swz<kBwdKeys>(16 * m + 4 * g + r, 16 * w + lo)] = sP[m][r];
    }
    if (kSplit) {
      // The next tile's copies complete (the partial's stores, issued after them, need not).
      if (p1_q0 >= 0 && wave_dq) {
        wait_vm<kPartStores>();
      } else {
        wait_mem();
      }
      __syncthreads();  // dS complete
    } else {
      // Stage 2's stores and the next tile's copies complete (stage 1's loads, issued last, may
      // still be in flight: they are needed only in the next iteration).
      if (p1_q0 >= 0 && p1_pos > 0 && wave_dq) {
        wait_vm<kStage1Loads>();
      } else {
        wait_mem();
      }
      __syncthreads();  // dS complete; every wave's stage-2 stores complete
      if (p2_q0 >= 0) pass_turn(p2_q0, p2_pos, p2_cnt);

      // Stages advance; this tile's dQ partial enters stage 1.
      p2_q0 = p1_q0;
      p2_pos = p1_pos;
      p2_cnt = p1_cnt;
#pragma unroll
      for (int j = 0; j < kDQ; ++j) {
#pragma unroll
        for (int m = 0; m < kNS; ++m) {
          p2[j][m] = p1[j][m];
#pragma unroll
          for (int r = 0; r < 4; ++r) p2s[j][m][r] = p1s[j][m][r];
        }
      }
    }
#pragma unroll
    for (int m = 0; m < kNS; ++m) {
#pragma unroll
      for (int j = 0; j < kDQ; ++j) p1[j][m] = zero4();
      if (q0 + 16 * m >= S || !wave_dq) continue;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const f4 x = ld4(&sdS[swz<kBwdKeys>(16 * m + lo, 16 * g + 4 * u)]);
#pragma unroll
        for (int j = 0; j < kDQ; ++j) {
          f4 y;
          if constexpr (kKtLds) {
            y = ld4(&sKt[(16 * (w + 4 * j) + lo) * kBwdLd + 16 * g + 4 * u]);
          } else {
            y = f4{kQ[j][4 * u], kQ[j][4 * u + 1], kQ[j][4 * u + 2], kQ[j][4 * u + 3]};
          }
          p1[j][m] = mma(x.x, y.x, p1[j][m]);
          p1[j][m] = mma(x.y, y.y, p1[j][m]);
          p1[j][m] = mma(x.z, y.z, p1[j][m]);
          p1[j][m] = mma(x.w, y.w, p1[j][m]);
        }
      }
    }
    p1_q0 = q0;
    p1_pos = pos_of(q0 / kQT);
    p1_cnt = count_of(q0 / kQT);
    // D of the next tile (its O and dO rows landed before the barrier above; the O buffer is
    // refilled only after the barrier below).
    if constexpr (kOwnD) {
      if (has_next) form_d(buf ^ 1);
    }
    __syncthreads();  // dS read by every wave
  };
  if constexpr (kSplit) {
    for (int t = 0; t < nsteps; t += 2) {
      tile_step(Const<0>{}, t);
      if (t + 1 < nsteps) tile_step(Const<1>{}, t + 1);
    }
  } else {
    for (int t = 0; t < nsteps; ++t) tile_step(Var{t & 1}, t);
  }

  // Drain: the tiles still in the pipeline, in order.
  if (kSplit) {
    if (p1_q0 >= 0) store_part(p1_q0, p1);
    if (a.arrive != nullptr) {
      // Every partial of this key block is stored once the stores of every wave have completed:
      // record its arrival, with the XCD it runs on (as bwd_split_kernel does).
      wait_stores();
      __syncthreads();
      if (tid == 0) {
        unsigned xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
        __hip_atomic_store(a.arrive + static_cast<int64_t>(bh) * a.nkb + kb, a.epoch | (xcc & 7u),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  } else if (p2_q0 >= 0) {
    store_sums(p2_q0, p2_pos, p2_cnt, p2, p2s);
    wait_stores();
    __syncthreads();
    pass_turn(p2_q0, p2_pos, p2_cnt);
  }
  if (!kSplit && p1_q0 >= 0) {
    load_sums(p1_q0, p1_pos, -1, p1s);
    store_sums(p1_q0, p1_pos, p1_cnt, p1, p1s);
    wait_stores();
    __syncthreads();
    pass_turn(p1_q0, p1_pos, p1_cnt);
  }

  // dK (x scale) and dV of this lane's key: dims 16 mt + 4 g .. + 3, one float4 each.
  if (key < S) {
    float* row = a.dqkv + (static_cast<int64_t>(b) * S + key) * 3 * a.H * D +
                 static_cast<int64_t>(h) * D;
    const int64_t part = static_cast<int64_t>(a.H) * D;
#pragma unroll
    for (int mt = 0; mt < kDT; ++mt) {
      st4(row + part + 16 * mt + 4 * g, dka[mt] * a.scale);
      st4(row + 2 * part + 16 * mt + 4 * g, dva[mt]);
    }
  }
  if constexpr (kSplit && kOwnSums) {
    if (a.causal && a.arrive != nullptr) {
      // The tiles whose last contributor is this key block (as bwd_split_kernel's).
      int j0, j1;
      own_tiles(kb, kBwdKeys, a.ntile, &j0, &j1);
      bwd_sum_range<D, kBwdKeys / kQT>(a, bh, j0, j1, &s_flag);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Backward, step 2 with the split dQ sum at D <= 64. The products, tile shapes, operand layouts and
// results are those of bwd_kernel<true, D> (the same operations in the same order, so the outputs
// are bit-identical); what changes is the schedule, which the split mode leaves free because no
// workgroup waits on another: one barrier per query tile instead of two. The staged tiles (Q, dO,
// O, L), D and dS have three LDS buffers (tile t in buffer t % 3). The copies of tile t + 2 are
// issued at the start of tile t and complete before tile t's barrier; after it, D of tile t + 2 is
// formed from its staged O and dO rows. So D of a tile is written two barriers before it is read,
// a tile's buffers are refilled only after the barrier that follows their last read, and a dS
// buffer is rewritten three tiles after it was written (its readers passed two barriers since).
// All LDS tiles sit in one array, so that each is a constant offset from one base: the compiler
// folds such offsets into the LDS instructions, where across separate arrays it keeps an address
// register per array (at D 64 that saves 24 registers).
// ---------------------------------------------------------------------------------------------
// dQ sums inside step 2 (split, D <= 64). Step 3 moves 118 MB at config 2 after step 2's tail,
// where the CUs run fewer and fewer key blocks; step 2 does those sums itself instead.
// bwd_sum_range sums query tiles j0 .. j1 - 1 of one (b, h) once every key block they need has
// finished. The partials are stored and loaded at device scope (st4_dev / ld4_dev: through to the
// coherence point that the XCDs share, whose L2s are not coherent with each other), so a sum may
// read partials that a key block on any XCD wrote. Each key block, once its partial stores have
// completed, writes the launch's epoch or'ed with its XCD to its arrival slot (a device-scope
// store, as the turn hand-over's counters). Wave 0 polls the (b, h)'s slots (device-scope loads)
// until every one it needs holds this launch's epoch, sleeping between polls. The sum is step 3's,
// operation for operation: float4 i of a tile's partials in key-block order, times scale (so the
// results are bit-identical whichever kernel sums a tile), stored from fragment order straight
// into dQ rows (16 lanes write 64 contiguous bytes). Then the tiles' done flags (the epoch), which
// step 3 checks when it runs: after a kernel-level step 2, while a graph is captured (step 3 also
// clears the flags a replay, with the same epoch, must not see), or where no sums are planned.
// Otherwise no step 3 follows (sums_final): a wait then gives up only after kSumPollsFinal polls
// (about a second), raising the guard word and writing NaN into the tiles' rows; with step 3 to
// follow it gives up after kSumPolls and leaves the tiles to step 3.
// Who sums:
//   non-causal: workgroups appended to step 2's grid (in-order dispatch starts them only once every
//   key block has been dispatched), kSumTiles query tiles each, every tile of every (b, h): those
//   on XCD x first take the (b, h)s whose last key block xcd_remap put on XCD x, in the order
//   their key blocks were dispatched, so the earliest sums wait for the earliest key blocks
//   (sum_plan / sum_target; the host sizes the grid from the same plan);
//   causal: key block kb's own workgroup, after its walk, sums the tiles whose last contributor it
//   is (own_tiles: its diagonal tiles 4 kb .. 4 kb + 3), which need key blocks 0 .. kb, whose
//   workgroups kb' b h + bh come earlier in the grid. No workgroup is appended: a tile is summed as
//   soon as its last key block finishes, while other key blocks still run, where summing
//   workgroups would start only after the last key block. At config 4 that is step 2 1202 -> 1116
//   us, at config 3 97.1 -> 93.6 us.
// Every poll ends: the key blocks waited for have smaller workgroup numbers, so they were
// dispatched before the polling workgroup and run to completion whatever it does.
// kSumTiles query tiles per summing workgroup: at config 2, 1, 2 or 15 were slower and 4 the same.
constexpr int kSumPolls = 4096;       // about 14 ms
constexpr int kSumPollsFinal = 1 << 18;  // about 0.9 s
template <int D, int NT>
__device__ __forceinline__ void bwd_sum_range(const BwdArgs& a, int bh, int j0, int j1,
                                              unsigned* flag) {
  constexpr int kDT = D / 16, kF4 = kQT * D / 4;
  const int tid = threadIdx.x, BH = a.nbh, ntile = a.ntile, nkb = a.nkb;
  // Key blocks whose partials the chunk needs: all, or (causal) those holding a key <= its last
  // query.
  const int need = a.causal ? min(nkb - 1, min(a.S - 1, j1 * kQT - 1) / a.kkeys) + 1 : nkb;
  if (tid < 64) {
    const unsigned long long* slots = a.arrive + static_cast<int64_t>(bh) * nkb;
    const int polls = a.bh0 + bh == a.give_up_bh ? 0 : a.sums_final ? kSumPollsFinal : kSumPolls;
    bool all = false;
    for (int it = 0; it < polls; ++it) {
      bool arrived = true;
      for (int kb = tid; kb < need; kb += 64) {
        const unsigned long long v =
            __hip_atomic_load(slots + kb, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        arrived = arrived && (v & ~7ull) == a.epoch;
      }
      if (__builtin_amdgcn_ballot_w64(!arrived) == 0) {
        all = true;
        break;
      }
      // About 1000 cycles between polls, 8000 after the first 256 (a sum dispatched while its
      // key blocks still have long to run: where they do not fill the chip).
      if (it < 256) {
        __builtin_amdgcn_s_sleep(16);
      } else {
        __builtin_amdgcn_s_sleep(127);
      }
    }
    if (tid == 0) *flag = all ? 1u : 0u;
    if (tid == 0 && !all && a.sums_final) {
      __hip_atomic_store(a.ctrl + kCtrlGuard, 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  const int b = (a.bh0 + bh) / a.H, h = (a.bh0 + bh) % a.H, S = a.S;
  const int64_t row_stride = static_cast<int64_t>(3) * a.H * D;
  float* const dq_bh =
      a.dqkv + static_cast<int64_t>(b) * S * row_stride + static_cast<int64_t>(h) * D;
  if (*flag == 0u) {
    if (a.sums_final) {
      // No step 3 follows: the tiles' dQ rows get NaN (the failure shows in the output).
      for (int e = tid; e < (j1 - j0) * kQT * D; e += kThreads) {
        const int q = j0 * kQT + e / D;
        if (q < S) dq_bh[q * row_stride + e % D] = __builtin_nanf("");
      }
    }
    return;
  }
  const int64_t slot = static_cast<int64_t>(BH) * ntile * (kQT * D);
  // Thread i sums float4 i (and i + kThreads, ... at D 128) of each of the tiles, four key blocks
  // at a time: the loads of all the tiles for those key blocks are issued together, then added in
  // key-block order.
  for (int i = tid; i < kF4; i += kThreads) {
    int cnt[NT];
    const float* src[NT];
    f4 acc[NT];
#pragma unroll
    for (int jj = 0; jj < NT; ++jj) {
      const int j = min(j0 + jj, j1 - 1);
      cnt[jj] = j0 + jj >= j1 ? 0
                : a.causal ? min(nkb - 1, min(S - 1, j * kQT + kQT - 1) / a.kkeys) + 1
                           : nkb;
      src[jj] = a.part + (static_cast<int64_t>(bh) * ntile + j) * (kQT * D);
    }
    for (int kb0 = 0; kb0 < need; kb0 += 4) {
      f4 x[NT][4];
#pragma unroll
      for (int jj = 0; jj < NT; ++jj) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int kb = kb0 + k;
          x[jj][k] = kb < cnt[jj]
                         ? ld4_dev(dev_rsrc(src[jj] + min(kb, cnt[jj] - 1) * slot, kQT * D * 4),
                                   16u * static_cast<unsigned>(i))
                         : zero4();
        }
      }
#pragma unroll
      for (int jj = 0; jj < NT; ++jj) {
        if (kb0 < cnt[jj]) acc[jj] = kb0 == 0 ? x[jj][0] : acc[jj] + x[jj][0];
#pragma unroll
        for (int k = 1; k < 4; ++k) {
          if (kb0 + k < cnt[jj]) acc[jj] += x[jj][k];
        }
      }
    }
    // Fragment order: register r of float4 i is query q0 + 16 mm + 4 g + r, dim 16 dt + lo.
    const int lane = i & 63, md = i >> 6, dt = md % kDT, mm = md / kDT;
    const int lo = lane & 15, g = lane >> 4;
#pragma unroll
    for (int jj = 0; jj < NT; ++jj) {
      if (j0 + jj >= j1) break;
      const f4 r4 = acc[jj] * a.scale;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int q = (j0 + jj) * kQT + 16 * mm + 4 * g + r;
        if (q < S) dq_bh[q * row_stride + 16 * dt + lo] = r4[r];
      }
    }
  }
  if (tid < j1 - j0) a.done[static_cast<int64_t>(bh) * ntile + j0 + tid] = a.epoch;
}

// A non-causal summing workgroup (m of XCD x).
template <int D>
__device__ __forceinline__ void bwd_sum_tiles(const BwdArgs& a, int x, int m, unsigned* flag) {
  int bh, j0;
  if (!sum_target(a.plan, (x + a.sum_shift) & 7, m, a.nbh, a.causal, &bh, &j0)) return;
  bwd_sum_range<D, kSumTiles>(a, bh, j0, min(a.ntile, j0 + kSumTiles), flag);
}

template <int D, int KG, bool kCausal>
__global__ void __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(KG == 1 || D == 32 ? BWD_WAVES : 2))) bwd_split_kernel(BwdArgs a) {
  // The mask is a compile-time constant of the instantiation (the host launches the one that
  // matches a.causal): every test of it below folds away (SGPR spills 19 -> 6 / 8 at D 64).
  a.causal = kCausal ? 1 : 0;
  constexpr int kKeys = kBwdKeys * KG;
  static_assert(D <= 64, "D 128 has no LDS room for three buffers: bwd_kernel<true, 128>");
  static_assert(kNS == 1, "one 16-query subtile per tile");
  constexpr int kKR = D / 4;                  // K (or V) values per lane: B operands of S, dP
  constexpr int kDT = D / 16;                 // 16-dim tiles (dK, dV accumulators; dQ tiles)
  constexpr int kCopies = kQT / kCopyRows<D>;  // direct copies per Q (or dO, O) tile
  constexpr int kNB = 3;                      // LDS buffers of the staged tiles, D and dS
  typedef float Tile[kQT * D];
  struct Smem {
    Tile q[kNB], g[kNB], o[kNB];
    float ds[kNB][kQT * kKeys];
    float l[kNB][kQT], d[kNB][kQT];
    unsigned flag;  // a dQ sum's poll result, from thread 0 to the workgroup
  };
  __shared__ __attribute__((aligned(16))) Smem sm;
  auto& sQ = sm.q;
  auto& sdO = sm.g;
  auto& sO = sm.o;
  auto& sdS = sm.ds;
  auto& sL = sm.l;
  auto& sD = sm.d;
  const unsigned lds0 = lds_addr(&sm);  // LDS byte address of the tiles

  const int tid = threadIdx.x, lane = tid & 63, lo = lane & 15, g = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in an SGPR
  const int BH = a.nbh, S = a.S;  // (b, h) local to this launch's chunk
  const int id = static_cast<int>(blockIdx.x);
  if (a.arrive != nullptr && id == 0 && tid == 0) *a.epoch_slot = a.epoch;  // for step 3
  if (a.arrive != nullptr && id >= a.nkb * BH) {
    // A dQ sum (the grid's last workgroups; those below n_main pad it to a multiple of 8).
    if (id >= a.n_main) bwd_sum_tiles<D>(a, id & 7, (id - a.n_main) >> 3, &sm.flag);
    return;
  }
  // The dQ product's 16-dim tiles: D / 16 of them for four waves. At D 64 wave w takes tile w on
  // every query tile; at D 32 waves 0, 1 take the two tiles on one query tile and waves 2, 3 on
  // the next (the turn alternating with the workgroup's parity as well), so that each SIMD gets
  // the same share of the products (with waves 0, 1 always, SIMDs 2, 3 idled a third of the
  // time at D 32). Who computes a fragment changes nothing in it.
  constexpr int kDqGroups = 4 / kDT;
  const int dt = w % kDT;
  auto dq_on = [&](int jt) { return kDqGroups == 1 || w / kDT == (jt + id) % kDqGroups; };
  // No turn waits here: the guard word reads 0 (unless a final sum's wait gave up; written
  // through, as that raise is, so that no copy of it lingers in this XCD's L2). Cleared by the
  // backward's first launch only: a backward split into chunks of (b, h) launches step 2 once per
  // chunk, and a later chunk must not clear what a sum of an earlier one raised.
  if (id == 0 && tid == 0 && a.bh0 == 0) {
    __hip_atomic_store(a.ctrl + kCtrlGuard, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // The key block: non-causal, (b, h)-major with the key blocks of one (b, h) on one XCD (they
  // read the same Q and dO tiles at about the same time); causal, key-block-major round-robin over
  // the XCDs (the expensive low blocks start first, spread evenly). Its walk: non-causal every
  // query tile, causal from the tile of the block's first key on.
  const int item = a.causal ? id : xcd_remap(id, a.nkb * BH);
  const int bh = a.causal ? item % BH : item / a.nkb;
  const int kb = a.causal ? item / BH : item % a.nkb;
  const int bhg = a.bh0 + bh;  // the (b, h) itself
  const int b = bhg / a.H, h = bhg % a.H;
  const int k0 = kb * kKeys;
  const int kw0 = k0 + 16 * KG * w;  // the wave's first key (KG groups of 16)
  const int key = kw0 + lo;          // this lane's key in group 0 (group c: + 16 c)
  const int t0 = a.causal ? k0 / kQT : 0;
  const int nsteps = a.ntile - t0;

  const float* qp = a.q.p + b * a.q.sb + h * a.q.sh;
  const float* kp = a.k.p + b * a.k.sb + h * a.k.sh;
  const float* vp = a.v.p + b * a.v.sb + h * a.v.sh;
  const float* gp = a.d_o.p + b * a.d_o.sb + h * a.d_o.sh;
  const float* op = a.o + (static_cast<int64_t>(b) * S * a.H + h) * D;
  const float* lp = a.lse + static_cast<int64_t>(bhg) * S;
  const unsigned q_ss4 = static_cast<unsigned>(a.q.ss) * 4u;
  const unsigned g_ss4 = static_cast<unsigned>(a.d_o.ss) * 4u;
  const unsigned o_ss4 = static_cast<unsigned>(a.H) * D * 4u;

  // K, V of this lane's key (B operands of S and dP) and kQ[t] = K[k0 + 16 g + t][16 w + lo]
  // (B operand of the dQ product), zero past S.
  // (Loads issued here; K and V are placed after the first tiles' copies are issued, below.)
  float kB[KG][kKR], vB[KG][kKR], kQ[KG][16];
  Quarter<D> kload[KG], vload[KG];
  {
#pragma unroll
    for (int c = 0; c < KG; ++c) {
      const int kr = min(key + 16 * c, S - 1);
      quarter_issue<D>(kp + kr * a.k.ss, g, kload[c]);
      quarter_issue<D>(vp + kr * a.v.ss, g, vload[c]);
    }
#pragma unroll
    for (int hh = 0; hh < KG; ++hh) {
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const int kk = k0 + 64 * hh + 16 * g + t;
        kQ[hh][t] = kk < S ? kp[min(kk, S - 1) * a.k.ss + 16 * dt + lo] : 0.0f;
      }
    }
  }

  // Staging of the query tile of walk step t into buffer `buf` (direct copies only; wave 0 copies
  // L): wave w issues copies w, w + 4, ... of the Q, dO and O tiles; rows past S repeat row S - 1.
  auto gload = [&](int t, auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    const int q0 = (t0 + t) * kQT;
#pragma unroll
    for (int j0 = 0; j0 < kCopies; j0 += 4) {
      if (j0 + w < kCopies) {
        copy_part_at<D>(qp, q_ss4, q0, S - 1, lds0 + offsetof(Smem, q[buf]), j0 + w, lane);
        copy_part_at<D>(gp, g_ss4, q0, S - 1, lds0 + offsetof(Smem, g[buf]), j0 + w, lane);
        copy_part_at<D>(op, o_ss4, q0, S - 1, lds0 + offsetof(Smem, o[buf]), j0 + w, lane);
      }
    }
    if (w == 0 && lane < kQT) {
      load_lds4_at(lp, 4u * static_cast<unsigned>(min(q0 + lane, S - 1)),
                   lds0 + offsetof(Smem, l[buf]));
    }
  };
  // D of the tile in buffer `buf` from its staged O and dO rows (as step 1: D / 4 lanes per row,
  // the same operations in the same order).
  auto rowsum_do_o = [&](auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    constexpr int kLanes = D / 4;
#pragma unroll
    for (int i0 = 0; i0 < kQT * kLanes; i0 += kThreads) {
      const int i = i0 + tid, row = i / kLanes, c4 = i % kLanes;
      float x = 0.0f;
      if (i < kQT * kLanes) {
        const f4 ov = ld4(&sO[buf][swz<D>(row, 4 * c4)]);
        const f4 gv = ld4(&sdO[buf][swz<D>(row, 4 * c4)]);
        x = ov.x * gv.x;
        x = fmaf(ov.y, gv.y, x);
        x = fmaf(ov.z, gv.z, x);
        x = fmaf(ov.w, gv.w, x);
      }
      x = lane_sum<kLanes>(x);
      if (i < kQT * kLanes && c4 == 0) sD[buf][row] = x;
    }
  };

  // The dQ partial of query tile j: the wave's 16 x 16 fragment (dim tile dt) in the key block's
  // slot, fragment order (register r of lane (lo, g) at 4 lane + r: query 16 j + 4 g + r, dim
  // 16 dt + lo); step 3 (dq_kernel) sums the slots.
  const float* const slot =
      a.part + (static_cast<int64_t>(kb) * BH + bh) * a.ntile * (kQT * D) + 256 * dt;

  f4 dva[KG][kDT], dka[KG][kDT];
#pragma unroll
  for (int c = 0; c < KG; ++c) {
#pragma unroll
    for (int mt = 0; mt < kDT; ++mt) {
      dva[c][mt] = zero4();
      dka[c][mt] = zero4();
    }
  }
  f4 p1 = zero4();  // the dQ fragment of the last tile (stored at the start of the next)
  auto store_frag = [&](int j) {
    st4_dev(dev_rsrc(slot + j * (kQT * D), 1024), 16u * static_cast<unsigned>(lane), p1);
  };

  gload(0, Const<0>{});
  if (nsteps > 1) gload(1, Const<1>{});
#pragma unroll
  for (int c = 0; c < KG; ++c) {
    quarter_place<D>(kload[c], kB[c]);
    quarter_place<D>(vload[c], vB[c]);
    if (kw0 + 16 * c + 16 > S) {  // wave-uniform: only a group with keys past S zeroes them
#pragma unroll
      for (int t = 0; t < kKR; ++t) {
        kB[c][t] = key + 16 * c < S ? kB[c][t] : 0.0f;
        vB[c][t] = key + 16 * c < S ? vB[c][t] : 0.0f;
      }
    }
  }
  wait_mem();  // the direct copies have landed
  __syncthreads();
  rowsum_do_o(Const<0>{});
  if (nsteps > 1) rowsum_do_o(Const<1>{});
  __syncthreads();

  auto tile_step = [&](auto bufc, int t) {
    constexpr int buf = decltype(bufc)::value;
    const int jt = t0 + t;  // query tile
    const int q0 = jt * kQT;
    // Tile t + 2 into the buffer of tile t - 1, whose last readers passed the last barrier.
    if (t + 2 < nsteps) gload(t + 2, Const<(buf + 2) % kNB>{});
    const bool frag_pending = t > 0 && dq_on(jt - 1);  // the last tile's fragment is unstored
    if (frag_pending) store_frag(jt - 1);
    compiler_fence();
    const float* Qt = sQ[buf];
    const float* Gt = sdO[buf];

    // Wave-uniform liveness of each group's 16 keys for the tile's 16 queries (a live group 1
    // implies a live group 0).
    bool live[KG];
    f4 sS[KG], sP[KG];
#pragma unroll
    for (int c = 0; c < KG; ++c) {
      const int kc = kw0 + 16 * c;
      live[c] = q0 < S && kc < S && !(a.causal && kc > q0 + 15);
      sS[c] = zero4();
      sP[c] = zero4();
    }
    if (live[0]) {
#pragma unroll
      for (int u = 0; u < kKR / 4; ++u) {
        const int at = swz<D>(lo, quarter_dim<D>(g, u));
        const f4 x = ld4(Qt + at), y = ld4(Gt + at);
#pragma unroll
        for (int c = 0; c < KG; ++c) {
          if (!live[c]) continue;
          sS[c] = mma(x.x, kB[c][4 * u], sS[c]);
          sS[c] = mma(x.y, kB[c][4 * u + 1], sS[c]);
          sS[c] = mma(x.z, kB[c][4 * u + 2], sS[c]);
          sS[c] = mma(x.w, kB[c][4 * u + 3], sS[c]);
          sP[c] = mma(y.x, vB[c][4 * u], sP[c]);
          sP[c] = mma(y.y, vB[c][4 * u + 1], sP[c]);
          sP[c] = mma(y.z, vB[c][4 * u + 2], sP[c]);
          sP[c] = mma(y.w, vB[c][4 * u + 3], sP[c]);
        }
      }
      const f4 Lv = ld4(&sL[buf][4 * g]), Dv = ld4(&sD[buf][4 * g]);
      const int qi0 = q0 + 4 * g;
#pragma unroll
      for (int c = 0; c < KG; ++c) {
        if (!live[c]) continue;
        const int kc = kw0 + 16 * c, keyc = key + 16 * c;
        if ((!a.causal || kc + 15 <= q0) && q0 + 16 <= S && kc + 16 <= S) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float p = exp2_hw(fmaf(sS[c][r], a.scale, -Lv[r]) * kLog2e);
            sP[c][r] = p * (sP[c][r] - Dv[r]);  // dS
            sS[c][r] = p;                        // P
          }
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const bool ok = qi0 + r < S && keyc < S && !(a.causal && keyc > qi0 + r);
            const float e = exp2_hw(fmaf(sS[c][r], a.scale, -Lv[r]) * kLog2e);
            const float p = ok ? e : 0.0f;
            sP[c][r] = p * (sP[c][r] - Dv[r]);  // dS
            sS[c][r] = p;                        // P
          }
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
#pragma unroll
        for (int mt = 0; mt < kDT; ++mt) {
          const int at = swz<D>(4 * g + r, 16 * mt + lo);
          const float gv = Gt[at], qv = Qt[at];
#pragma unroll
          for (int c = 0; c < KG; ++c) {
            if (!live[c]) continue;
            dva[c][mt] = mma(gv, sS[c][r], dva[c][mt]);
            dka[c][mt] = mma(qv, sP[c][r], dka[c][mt]);
          }
        }
      }
    }

    // This tile's dS into LDS (zero where a group's keys are all masked).
#pragma unroll
    for (int c = 0; c < KG; ++c) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sdS[buf][swz<kKeys>(4 * g + r, 16 * (KG * w + c) + lo)] = sP[c][r];
      }
    }
    if (frag_pending) {
      wait_vm<1>();  // tile t + 2's copies complete (the fragment's store, issued after, need not)
    } else {
      wait_mem();
    }
    __syncthreads();  // dS complete; tile t + 2's rows landed

    // The dQ partial dS K over the block's keys (the wave's dim tile dt, if its turn).
    p1 = zero4();
    if (q0 < S && dq_on(jt)) {
#pragma unroll
      for (int hh = 0; hh < KG; ++hh) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const f4 x = ld4(&sdS[buf][swz<kKeys>(lo, 64 * hh + 16 * g + 4 * u)]);
          p1 = mma(x.x, kQ[hh][4 * u], p1);
          p1 = mma(x.y, kQ[hh][4 * u + 1], p1);
          p1 = mma(x.z, kQ[hh][4 * u + 2], p1);
          p1 = mma(x.w, kQ[hh][4 * u + 3], p1);
        }
      }
    }
    // D of tile t + 2 (its rows landed before the barrier).
    if (t + 2 < nsteps) rowsum_do_o(Const<(buf + 2) % kNB>{});
  };
  // Unrolled by three, so that every LDS buffer index is a compile-time constant.
  for (int t = 0; t < nsteps; t += 3) {
    tile_step(Const<0>{}, t);
    if (t + 1 < nsteps) tile_step(Const<1>{}, t + 1);
    if (t + 2 < nsteps) tile_step(Const<2>{}, t + 2);
  }
  if (dq_on(t0 + nsteps - 1)) store_frag(t0 + nsteps - 1);  // the last tile's fragment
  if (a.arrive != nullptr) {
    // Every partial of this key block is stored once the stores of every wave have completed:
    // record its arrival, with the XCD it runs on (dK and dV, stored below, are not read by the
    // sums).
    wait_mem();
    __syncthreads();
    if (tid == 0) {
      unsigned xcc;
      asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
      __hip_atomic_store(a.arrive + static_cast<int64_t>(bh) * a.nkb + kb, a.epoch | (xcc & 7u),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  // dK (x scale) and dV of this lane's keys: dims 16 mt + 4 g .. + 3, one float4 each.
#pragma unroll
  for (int c = 0; c < KG; ++c) {
    const int keyc = key + 16 * c;
    if (keyc < S) {
      float* row = a.dqkv + (static_cast<int64_t>(b) * S + keyc) * 3 * a.H * D +
                   static_cast<int64_t>(h) * D;
      const int64_t part = static_cast<int64_t>(a.H) * D;
#pragma unroll
      for (int mt = 0; mt < kDT; ++mt) {
        st4(row + part + 16 * mt + 4 * g, dka[c][mt] * a.scale);
        st4(row + 2 * part + 16 * mt + 4 * g, dva[c][mt]);
      }
    }
  }
  if (a.causal && a.arrive != nullptr) {
    // The tiles whose last contributor is this key block (the summing workgroups' work, causal).
    int j0, j1;
    own_tiles(kb, kKeys, a.ntile, &j0, &j1);
    bwd_sum_range<D, kKeys / kQT>(a, bh, j0, j1, &sm.flag);
  }
}

// ---------------------------------------------------------------------------------------------
// Backward, step 3 (split only): dQ of a (b, h, query tile), the tile's partials summed in
// key-block order, ((p_0 + p_1) + p_2) + ..., times scale (the same operations, in the same order,
// as the turn hand-over and as step 2's own sums). Float4 i of a partial (fragment order: dim tile
// dt = i / 64 of subtile m, lane l = i % 64, registers r = 0..3 -> query 16 m + 4 (l / 16) + r,
// dim 16 dt + l % 16) is summed by one thread, then the tile goes through LDS so that every row of
// dQ is written as D / 4 float4s.
// ---------------------------------------------------------------------------------------------
template <int D>
__device__ __forceinline__ void dq_tile(const float* __restrict__ part, float* __restrict__ dqkv,
                                        int nbh, int bh0, int H, int S, int nkb, int ntile,
                                        float scale, int causal, int bh, int j, float* tile,
                                        int kkeys) {
  constexpr int kDT = D / 16, kPitch = D + 4;  // pitch: conflict-free fragment writes
  constexpr int kF4 = kQT * D / 4;             // float4s per tile
  const int tid = threadIdx.x;
  const int b = (bh0 + bh) / H, h = (bh0 + bh) % H, q0 = j * kQT;
  // Contributors: causal, the key blocks holding a key <= the tile's last query.
  const int cnt = causal ? min(nkb - 1, min(S - 1, q0 + kQT - 1) / kkeys) + 1 : nkb;
  const int64_t slot = static_cast<int64_t>(nbh) * ntile * (kQT * D);
  const float* src = part + (static_cast<int64_t>(bh) * ntile + j) * (kQT * D);
#pragma unroll
  for (int i = tid; i < kF4; i += kThreads) {
    // Loads four slots at a time (independent), adds them in key-block order.
    f4 acc = ld4(src + 4 * i);
    int kb = 1;
    for (; kb + 3 < cnt; kb += 4) {
      const f4 x0 = ld4(src + kb * slot + 4 * i), x1 = ld4(src + (kb + 1) * slot + 4 * i);
      const f4 x2 = ld4(src + (kb + 2) * slot + 4 * i), x3 = ld4(src + (kb + 3) * slot + 4 * i);
      acc += x0;
      acc += x1;
      acc += x2;
      acc += x3;
    }
    for (; kb < cnt; ++kb) acc += ld4(src + kb * slot + 4 * i);
    acc *= scale;
    const int lane = i & 63, md = i >> 6, dt = md % kDT, m = md / kDT;
    const int lo = lane & 15, g = lane >> 4;
#pragma unroll
    for (int r = 0; r < 4; ++r) tile[(16 * m + 4 * g + r) * kPitch + 16 * dt + lo] = acc[r];
  }
  __syncthreads();
#pragma unroll
  for (int i = tid; i < kF4; i += kThreads) {
    const int row = i / (D / 4), c4 = i % (D / 4);
    if (q0 + row < S) {
      st4(dqkv + (static_cast<int64_t>(b) * S + q0 + row) * 3 * H * D +
              static_cast<int64_t>(h) * D + 4 * c4,
          ld4(&tile[row * kPitch + 4 * c4]));
    }
  }
}

// One workgroup per query tile (done == null), or, after step 2's own sums, each workgroup checks
// a range of up to kThreads tiles (one flag per thread) and sums those whose flag does not hold
// the epoch of the step 2 launch (recorded in the workspace), one after the other. It then zeroes
// the flags it read and a range of the key blocks' arrival slots: every backward leaves that state
// clear, so a launch whose epoch repeats (a replayed graph bakes in its launch arguments) never
// meets its own earlier values.
template <int D>
__global__ void __launch_bounds__(kThreads) dq_kernel(const float* __restrict__ part,
                                                     unsigned long long* __restrict__ done,
                                                     unsigned long long* __restrict__ arrive,
                                                     const unsigned long long* __restrict__ epoch,
                                                     float* __restrict__ dqkv, int nbh, int bh0,
                                                     int H, int S, int nkb, int ntile,
                                                     float scale, int causal, int kkeys) {
  __shared__ __attribute__((aligned(16))) float tile[kQT * (D + 4)];
  __shared__ int todo[kThreads];
  __shared__ int ntodo;
  const int tot = nbh * ntile;  // this launch's (b, h) chunk
  if (done == nullptr) {
    // Non-causal: the tiles of a (b, h) on the XCD that ran its key blocks in step 2 (the same
    // XCD-major split of the grid), the (b, h) written last first, whose partials are likeliest
    // still cached.
    int it = static_cast<int>(blockIdx.x);
    if (!causal && it < (tot & ~7)) it = (it & 7) * (tot >> 3) + ((tot >> 3) - 1 - (it >> 3));
    dq_tile<D>(part, dqkv, nbh, bh0, H, S, nkb, ntile, scale, causal, it / ntile, it % ntile,
               tile, kkeys);
    return;
  }
  const int tid = threadIdx.x;
  const int per = (tot + static_cast<int>(gridDim.x) - 1) / static_cast<int>(gridDim.x);
  const int first = static_cast<int>(blockIdx.x) * per, n = min(per, tot - first);
  if (tid == 0) ntodo = 0;
  __syncthreads();
  if (tid < n) {
    if (done[first + tid] != *epoch) todo[atomicAdd(&ntodo, 1)] = first + tid;
    done[first + tid] = 0ull;
  }
  const int nslot = nbh * nkb;
  const int per_slot = (nslot + static_cast<int>(gridDim.x) - 1) / static_cast<int>(gridDim.x);
  const int slot0 = static_cast<int>(blockIdx.x) * per_slot;
  if (tid < min(per_slot, nslot - slot0)) arrive[slot0 + tid] = 0ull;
  __syncthreads();
  const int k = ntodo;
  for (int i = 0; i < k; ++i) {
    const int it = todo[i];
    dq_tile<D>(part, dqkv, nbh, bh0, H, S, nkb, ntile, scale, causal, it / ntile, it % ntile,
               tile, kkeys);
    __syncthreads();  // the LDS tile is reused
  }
}

}  // namespace

// Forward shapes per head_dim and mask: queries per workgroup, keys per tile, waves per SIMD
// (D 128: two; 16-key tiles, 32 KB of LDS per workgroup: at b 64 h 6 s 240 non-causal 106.5 us
// against 113.3 for 32-key tiles, at b 8 h 12 s 2048 causal 801.5 against 830.2).
template <int D, int C>
struct FwdCfg;
template <>
struct FwdCfg<32, 0> {
  static constexpr int QB = 128, KT = 64, W = 3;
};
template <>
struct FwdCfg<32, 1> {
  static constexpr int QB = 64, KT = 32, W = 3;
};
template <>
struct FwdCfg<64, 0> {
  static constexpr int QB = 128, KT = 32, W = 3;
};
template <>
struct FwdCfg<64, 1> {
  static constexpr int QB = 64, KT = 32, W = 3;
};
template <>
struct FwdCfg<128, 0> {
  static constexpr int QB = 64, KT = 16, W = 2;
};
template <>
struct FwdCfg<128, 1> {
  static constexpr int QB = 64, KT = 16, W = 2;
};
// D 32 non-causal over short sequences takes 48-key tiles where they leave fewer padded keys than
// 64-key tiles: up to s 512 the last, masked tile is an eighth of the walk or more. Measured
// (forward, d 32, 48-key against 64-key tiles): s 240 -2.7 to -4.7 %, 336 -3.4 %, 480 -1.4 %, 200
// -1.1 %; with equal padding 64 keys win (s 192 +2.0 %, 384 +1.0 %), and on long sequences the
// last tile weighs less (s 720 +0.2 %, 2000 +1.0 %).
constexpr int kFwdShortKeys32 = 48;
constexpr int kFwdShortMaxS32 = 512;
static bool fwd_short_tiles32(int64_t s) {
  constexpr int kLong = FwdCfg<32, 0>::KT, kShort = kFwdShortKeys32;
  const int64_t pad_long = (s + kLong - 1) / kLong * kLong - s;
  const int64_t pad_short = (s + kShort - 1) / kShort * kShort - s;
  return s <= kFwdShortMaxS32 && pad_short < pad_long;
}

namespace {

template <int D, int C>
const void* fwd_fn() {
  using F = FwdCfg<D, C>;
  return reinterpret_cast<const void*>(fwd_kernel<D, F::QB, F::KT, F::W, C != 0>);
}

// Step 2's split kernel for 64-key (or, `wide`, 128-key) blocks and the mask; causal runs 64-key
// blocks only (bwd_split_keys), so a wide causal request has no kernel.
template <int D>
const void* split_fn(bool wide, bool causal) {
  if (wide) return causal ? nullptr : reinterpret_cast<const void*>(bwd_split_kernel<D, 2, false>);
  return causal ? reinterpret_cast<const void*>(bwd_split_kernel<D, 1, true>)
                : reinterpret_cast<const void*>(bwd_split_kernel<D, 1, false>);
}

int fwd_qb(int d, int causal) {
  const int c = causal ? 1 : 0;
  switch (d) {
    case 32: return c ? FwdCfg<32, 1>::QB : FwdCfg<32, 0>::QB;
    case 128: return c ? FwdCfg<128, 1>::QB : FwdCfg<128, 0>::QB;
    default: return c ? FwdCfg<64, 1>::QB : FwdCfg<64, 0>::QB;
  }
}

hipError_t launch(const void* fn, int64_t blocks, void** args, void* stream) {
  return hipLaunchKernel(fn, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), args, 0,
                         static_cast<hipStream_t>(stream));
}

}  // namespace

bool head_dim_supported(int64_t d) { return d == 32 || d == 64 || d == 128; }

int64_t forward_blocks(int64_t b, int64_t h, int64_t s, int causal, int d) {
  const int qb = fwd_qb(d, causal);
  return ((s + qb - 1) / qb) * h * b;
}
int64_t bwd_main_blocks(int64_t b, int64_t h, int64_t s) {
  return ((s + kBwdKeys - 1) / kBwdKeys) * h * b;
}
int64_t bwd_prep_blocks(int64_t b, int64_t h, int64_t s, int d) {
  const int64_t rows_per_block = kThreads / (d / 4);
  return (b * h * s + rows_per_block - 1) / rows_per_block;
}
int64_t bwd_dq_blocks(int64_t b, int64_t h, int64_t s) { return b * h * ((s + kQT - 1) / kQT); }
bool bwd_own_d(int64_t s, int d) {
  // D 128 split: step 2 forms D itself up to kOwnDMaxBlocks key blocks per (b, h), where every
  // key block re-forming D for its tiles costs less than step 1's launch and pass over O and dO.
  // Measured (backward, A/B in one process): b 64 h 6 s 240 320.9 -> 314.7 us, causal 230.4 ->
  // 228.9; but b 8 h 12 s 2048 causal 2334 -> 2490 and b 16 h 16 s 1024 3052 -> 3186.
  return d == 128 && (s + kBwdKeys - 1) / kBwdKeys <= kOwnDMaxBlocks;
}
bool bwd_needs_prep(bool split, int d, int64_t s) {
  return !split || (d > 64 && !bwd_own_d(s, d));
}
namespace {
std::atomic<int> g_step2_sums{1};
std::atomic<int> g_sum_shift{0};
std::atomic<int> g_give_up_bh{-1};
}  // namespace
bool set_step2_sums(bool on) { return g_step2_sums.exchange(on ? 1 : 0) != 0; }
int set_sum_shift(int shift) { return g_sum_shift.exchange(shift & 7); }
int set_give_up_bh(int bh) { return g_give_up_bh.exchange(bh < 0 ? -1 : bh); }
void test_hook_state(int64_t out[3]) {
  out[0] = g_step2_sums.load(std::memory_order_relaxed);
  out[1] = g_sum_shift.load(std::memory_order_relaxed);
  out[2] = g_give_up_bh.load(std::memory_order_relaxed);
}

int bwd_split_keys(int64_t b, int64_t h, int64_t s, int d, int causal) {
  // 128-key blocks (two 16-key groups per wave): half the dQ partials and half the per-tile
  // staging and barriers per product. At d 64 they hold 2 waves per SIMD instead of 3. Measured
  // (step 2, non-causal, d 64): s 384 +3.9 %, 512 -4.8 %, 768 -4.1 %, 1024 -6.7 %, 2048 -6.9 %,
  // 4096 -3.6 %; causal +1 to +31 % (the diagonal blocks' masked work doubles). They need two
  // workgroups per CU to fill the chip. At d 32 they keep 3 waves per SIMD and pay where the
  // halved workgroup count leaves fewer than two rounds of them (b h s 256 +8 %, 512 +60 %,
  // config 2's shape -2 %); from two rounds on (1536 workgroups) they gain: b16 h16 s768 -3.4 %,
  // s1024 -5.0 %, b8 h16 s2048 -4.4 %, b4 h16 s4096 -4.2 %.
  const int64_t blocks128 = (s + 2 * kBwdKeys - 1) / (2 * kBwdKeys) * b * h;
  if (causal) return kBwdKeys;
  if (d == 32) return blocks128 >= 1536 ? 2 * kBwdKeys : kBwdKeys;
  if (d != 64 || s < 512) return kBwdKeys;
  return blocks128 >= 512 ? 2 * kBwdKeys : kBwdKeys;
}
namespace {
// The schedule of a launch over nbh (b, h) pairs with key blocks of `keys` keys (a chunk's keys
// come from the whole launch's pair count: every chunk has the whole's arithmetic).
bool step2_sums_of(int64_t nbh, int64_t s, int d, int causal, int keys) {
  if (g_step2_sums.load(std::memory_order_relaxed) == 0) return false;
  // The range check keeps b h s (hence every count below) inside int32.
  const int nkb = static_cast<int>((s + keys - 1) / keys);
  const int ntile = static_cast<int>((s + kQT - 1) / kQT);
  return sum_plan(static_cast<int>(nbh), nkb, ntile, d, causal).on != 0;
}
int64_t sum_blocks_of(int64_t nbh, int64_t s, int d, int causal, int keys) {
  if (causal || !step2_sums_of(nbh, s, d, causal, keys)) return 0;
  const int nkb = static_cast<int>((s + keys - 1) / keys);
  const int ntile = static_cast<int>((s + kQT - 1) / kQT);
  const SumPlan p = sum_plan(static_cast<int>(nbh), nkb, ntile, d, causal);
  return sum_blocks(p, static_cast<int>(nbh), causal);
}
int64_t dq_grid_of(int64_t nbh, int64_t s, int d, int causal, int keys) {
  const int64_t tiles = bwd_dq_blocks(1, nbh, s);
  if (!step2_sums_of(nbh, s, d, causal, keys)) return tiles;
  const int64_t g = std::max<int64_t>(256, (tiles + kThreads - 1) / kThreads);
  return std::min(tiles, g);
}
}  // namespace
bool bwd_step2_sums_all(int64_t nbh, int64_t b, int64_t h, int64_t s, int d, int causal) {
  // The plan, where on, gives every query tile of every (b, h) to one summing unit.
  const int keys = d <= 64 ? bwd_split_keys(b, h, s, d, causal) : kBwdKeys;
  return step2_sums_of(nbh, s, d, causal, keys);
}
bool bwd_step2_sums(int64_t b, int64_t h, int64_t s, int d, int causal) {
  return step2_sums_of(b * h, s, d, causal, bwd_split_keys(b, h, s, d, causal));
}
int64_t bwd_sum_blocks(int64_t b, int64_t h, int64_t s, int d, int causal) {
  return sum_blocks_of(b * h, s, d, causal, bwd_split_keys(b, h, s, d, causal));
}
int64_t bwd_dq_grid(int64_t b, int64_t h, int64_t s, int d, int causal) {
  return dq_grid_of(b * h, s, d, causal, bwd_split_keys(b, h, s, d, causal));
}


int launch_forward(View q, View k, View v, float* o, float* lse, int b, int h, int s, int d,
                   float scale, int causal, void* stream) {
  const int c = causal ? 1 : 0;
  const int qb = fwd_qb(d, c);
  FwdArgs a{q, k, v, o, lse, b, h, s, (s + qb - 1) / qb, scale, c};
  void* args[] = {&a};
  const void* fn32 =
      c ? fwd_fn<32, 1>()
      : fwd_short_tiles32(s)
          ? reinterpret_cast<const void*>(
                fwd_kernel<32, FwdCfg<32, 0>::QB, kFwdShortKeys32, FwdCfg<32, 0>::W, false>)
          : fwd_fn<32, 0>();
  const void* fn = d == 32    ? fn32
                   : d == 128 ? (c ? fwd_fn<128, 1>() : fwd_fn<128, 0>())
                              : (c ? fwd_fn<64, 1>() : fwd_fn<64, 0>());
  return static_cast<int>(launch(fn, forward_blocks(b, h, s, c, d), args, stream));
}

int launch_bwd_prep(const float* o, View d_o, float* dsum, int* turn, int* ctrl, int b, int h,
                    int s, int d, void* stream) {
  int nturn = b * h * ((s + kQT - 1) / kQT);
  void* args[] = {&o, &d_o, &dsum, &turn, &ctrl, &b, &h, &s, &nturn};
  const void* fn = d == 32    ? reinterpret_cast<const void*>(prep_kernel<32>)
                   : d == 128 ? reinterpret_cast<const void*>(prep_kernel<128>)
                              : reinterpret_cast<const void*>(prep_kernel<64>);
  return static_cast<int>(launch(fn, bwd_prep_blocks(b, h, s, d), args, stream));
}

int launch_bwd_main(View q, View k, View v, View d_o, const float* o, const float* lse,
                    const float* dsum, float* dqkv, float* part, unsigned long long* arrive,
                    unsigned long long* done, unsigned long long* epoch_slot,
                    unsigned long long epoch, int* turn, int* ctrl, int b, int h, int s, int d,
                    float scale, int causal, int bh0, int nbh, int sums_final,
                    void* stream) {
  int nkb = (s + kBwdKeys - 1) / kBwdKeys, ntile = (s + kQT - 1) / kQT;
  const bool split = part != nullptr;
  // The split path's grid is that of the chunk (nbh pairs) with the whole's key blocks; the
  // turn path covers all pairs.
  if (!split || d > 64) bh0 = 0, nbh = b * h;
  const int kkeys = split && d <= 64 ? bwd_split_keys(b, h, s, d, causal) : kBwdKeys;
  nkb = (s + kkeys - 1) / kkeys;
  const int stagger = !split && !causal && nkb <= kStaggerMaxBlocks ? 1 : 0;
  const int64_t nsum = split ? sum_blocks_of(nbh, s, d, causal, kkeys) : 0;
  const int64_t nblk = int64_t{nkb} * nbh;
  const int64_t nmain = (nblk + 7) & ~int64_t{7};
  if (!split || !step2_sums_of(nbh, s, d, causal, kkeys)) {
    arrive = nullptr, done = nullptr, epoch_slot = nullptr;
  }
  const SumPlan plan = sum_plan(nbh, nkb, ntile, d, causal);
  BwdArgs a{q,    k,     v,    d_o,  o,    lse,   dsum,       dqkv,  part,
            arrive, done, epoch_slot, epoch, static_cast<int>(nmain), plan, turn, ctrl, b, h, s,
            nkb,  ntile, scale, causal, stagger, kkeys, bh0, nbh,
            arrive != nullptr && sums_final ? 1 : 0, g_sum_shift.load(std::memory_order_relaxed),
            g_give_up_bh.load(std::memory_order_relaxed)};
  void* args[] = {&a};
  if (split && d <= 64) {
    const bool wide = kkeys != kBwdKeys;
    const void* fn = d == 32 ? split_fn<32>(wide, causal) : split_fn<64>(wide, causal);
    if (fn == nullptr) return static_cast<int>(hipErrorInvalidValue);
    return static_cast<int>(launch(fn, nsum ? nmain + nsum : nblk, args, stream));
  }
  // The turn mode at every head_dim; the split mode at 128 (no LDS room for bwd_split_kernel).
  const bool own_d = split && bwd_own_d(s, d);
  const void* fn;
  if (d == 32) {
    fn = reinterpret_cast<const void*>(bwd_kernel<false, 32>);
  } else if (d == 128) {
    fn = !split  ? reinterpret_cast<const void*>(bwd_kernel<false, 128>)
         : causal ? (own_d ? reinterpret_cast<const void*>(bwd_kernel<true, 128, true, true>)
                           : reinterpret_cast<const void*>(bwd_kernel<true, 128, true>))
                  : (own_d ? reinterpret_cast<const void*>(bwd_kernel<true, 128, false, true>)
                           : reinterpret_cast<const void*>(bwd_kernel<true, 128>));
  } else {
    fn = reinterpret_cast<const void*>(bwd_kernel<false, 64>);
  }
  // (Split at 128: the key blocks, then the workgroups of the tail sums, as above.)
  if (split) return static_cast<int>(launch(fn, nsum ? nmain + nsum : nblk, args, stream));
  return static_cast<int>(launch(fn, bwd_main_blocks(b, h, s), args, stream));
}

// The device address of `scratch` on the device that runs `stream` (the null stream: the current
// device), looked up with hipGetSymbolAddress once per device, with that device current, and kept.
int static_scratch(void* stream, void** out) {
  constexpr int kMaxDevices = 64;
  static std::atomic<void*> addr[kMaxDevices];
  static std::mutex mu;
  int dev = 0;
  hipError_t e = stream ? hipStreamGetDevice(static_cast<hipStream_t>(stream), &dev)
                        : hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return static_cast<int>(hipErrorInvalidDevice);
  void* p = addr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(mu);
    p = addr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      int cur = 0;
      if ((e = hipGetDevice(&cur)) != hipSuccess) return static_cast<int>(e);
      if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return static_cast<int>(e);
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (cur != dev) {
        const hipError_t e2 = hipSetDevice(cur);
        if (e == hipSuccess) e = e2;
      }
      if (e != hipSuccess) return static_cast<int>(e);
      if (p == nullptr) return static_cast<int>(hipErrorInvalidSymbol);
      addr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return 0;
}

int launch_bwd_dq(const float* part, unsigned long long* done, unsigned long long* arrive,
                  const unsigned long long* epoch_slot, float* dqkv, int b, int h, int s, int d,
                  float scale, int causal, int bh0, int nbh, void* stream) {
  if (d > 64) bh0 = 0, nbh = b * h;  // (the split path at d 128 is not chunked)
  int kkeys = bwd_split_keys(b, h, s, d, causal);
  int nkb = (s + kkeys - 1) / kkeys, ntile = (s + kQT - 1) / kQT;
  if (!step2_sums_of(nbh, s, d, causal, kkeys)) {
    done = nullptr, arrive = nullptr, epoch_slot = nullptr;
  }
  void* args[] = {&part, &done, &arrive, &epoch_slot, &dqkv,  &nbh,    &bh0,
                  &h,    &s,    &nkb,    &ntile,      &scale, &causal, &kkeys};
  const void* fn = d == 32    ? reinterpret_cast<const void*>(dq_kernel<32>)
                   : d == 128 ? reinterpret_cast<const void*>(dq_kernel<128>)
                              : reinterpret_cast<const void*>(dq_kernel<64>);
  return static_cast<int>(launch(fn, dq_grid_of(nbh, s, d, causal, kkeys), args, stream));
}

}  // namespace fattn
