// Fused fp32 scaled-dot-product attention for gfx950 (MI355X / CDNA4), head_dim 64: a
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
// seq) strides with head_dim contiguous, every row 16-byte aligned; O is written [b, s, h, 64];
// L and D are [b, h, s]; dQ, dK, dV are written interleaved into one [b, s, 3, h, 64] buffer.
//
// Determinism: every sum has an order fixed by the shape alone. The cross-workgroup sum (dQ over
// key blocks) is done in key-block order under one turn counter per (b, h, query tile); key blocks
// are handed out by a ticket in arrival order, so a workgroup only ever waits on a key block that a
// running workgroup already holds (no assumption about dispatch order).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "fattn_internal.h"

namespace fattn {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;  // 4 waves of 64
constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kNegInf = -__builtin_inff();
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
__device__ __forceinline__ f4 zero4() { return f4{0.0f, 0.0f, 0.0f, 0.0f}; }

// Workgroups are handed to the 8 XCDs round-robin (id % 8). This permutation gives each XCD a
// contiguous range of logical indices, so logical neighbours (same (b, h)) share one L2.
__device__ __forceinline__ int xcd_remap(int id, int total) {
  const int full = total & ~7;
  if (id >= full) return id;
  return (id & 7) * (full >> 3) + (id >> 3);
}

// ---------------------------------------------------------------------------------------------
// Forward. One workgroup = 64 queries of one (b, h); wave w owns queries q0 + 16 w .. + 15, one
// per lane column lo. Key tiles of 64 are staged in LDS (double buffered, the next tile's loads in
// flight during this tile's math) and shared by the four waves.
//   S^T = K Q^T per 16-key subtile: A = K[key 16 mt + lo][dim 16 g + t] (LDS, float4 reads),
//   B = Q[query lo][dim 16 g + t] (registers, loaded once). Output: lane (lo, g) holds
//   S[query lo][key 16 mt + 4 g + r].
//   O^T += V^T P^T: M = dims (four 16-row tiles), N = queries, contraction over the tile's keys;
//   step (kt, r) uses key 16 kt + 4 g + r, i.e. exactly the P value lane (lo, g) holds in its
//   register (kt, r). A = V[key][dim 16 mt + lo] (LDS).
// Online softmax per query: running max m (identical in the four lanes of the query), running
// partial sum over the lane's own keys (combined across the four lanes once, in a fixed order,
// at the end), O rescaled by alpha = exp(m_old - m_new) when the max grows.
// ---------------------------------------------------------------------------------------------
constexpr int kFwdWaveQ = 16;
constexpr int kFwdKeys = 64;
constexpr int kFwdLd = 68;  // LDS row pitch (floats): conflict-free float4 and column reads

struct FwdArgs {
  View q, k, v;
  float* o;
  float* lse;
  int B, H, S, nqb;
  float scale;
  int causal;
};

__global__ void __launch_bounds__(kThreads) fwd_kernel(FwdArgs a) {
  __shared__ __attribute__((aligned(16))) float sK[2][kFwdKeys * kFwdLd];
  __shared__ __attribute__((aligned(16))) float sV[2][kFwdKeys * kFwdLd];

  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, lo = lane & 15, g = lane >> 4;
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
  const int qi = qw0 + lo;             // this lane's query
  const float* qp = a.q.p + b * a.q.sb + h * a.q.sh;
  const float* kp = a.k.p + b * a.k.sb + h * a.k.sh;
  const float* vp = a.v.p + b * a.v.sb + h * a.v.sh;

  // B operand of S^T: Q[qi][16 g .. 16 g + 15].
  float qr[16];
  if (qi < S) {
    const float* r = qp + qi * a.q.ss + 16 * g;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const f4 x = ld4(r + 4 * u);
      qr[4 * u] = x.x;
      qr[4 * u + 1] = x.y;
      qr[4 * u + 2] = x.z;
      qr[4 * u + 3] = x.w;
    }
  } else {
#pragma unroll
    for (int t = 0; t < 16; ++t) qr[t] = 0.0f;
  }

  // Keys the block needs, and keys this wave's rows can see.
  const int k_end = a.causal ? min(S, q0 + kFwdQueries) : S;
  const int ntiles = (k_end + kFwdKeys - 1) / kFwdKeys;
  const int kw_end = a.causal ? min(S, qw0 + kFwdWaveQ) : S;
  const bool wave_live = qw0 < S;

  // Staging: thread tid moves rows (tid / 16) + 16 i, float4 column tid % 16, of K and V.
  const int srow = tid >> 4, sc4 = tid & 15;
  f4 kst[4], vst[4];
  auto gload = [&](int kt0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = kt0 + srow + 16 * i;
      if (key < S) {
        kst[i] = ld4(kp + key * a.k.ss + 4 * sc4);
        vst[i] = ld4(vp + key * a.v.ss + 4 * sc4);
      } else {  // zero rows: masked scores, and 0 * V must stay 0
        kst[i] = zero4();
        vst[i] = zero4();
      }
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      st4(&sK[buf][(srow + 16 * i) * kFwdLd + 4 * sc4], kst[i]);
      st4(&sV[buf][(srow + 16 * i) * kFwdLd + 4 * sc4], vst[i]);
    }
  };

  f4 acc[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) acc[mt] = zero4();
  float m = kNegInf, lsum = 0.0f;

  gload(0);
  sstore(0);
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1, kt0 = t * kFwdKeys;
    const bool has_next = t + 1 < ntiles;
    if (has_next) gload(kt0 + kFwdKeys);  // in flight during this tile's math
    if (wave_live) {
      const float* Kt = sK[buf];
      const float* Vt = sV[buf];
      bool live[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) live[mt] = kt0 + 16 * mt < kw_end;  // wave-uniform
      f4 s[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        s[mt] = zero4();
        if (live[mt]) {
          const float* kr = Kt + (16 * mt + lo) * kFwdLd + 16 * g;
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const f4 kk = ld4(kr + 4 * u);
            s[mt] = mma(kk.x, qr[4 * u], s[mt]);
            s[mt] = mma(kk.y, qr[4 * u + 1], s[mt]);
            s[mt] = mma(kk.z, qr[4 * u + 2], s[mt]);
            s[mt] = mma(kk.w, qr[4 * u + 3], s[mt]);
          }
        }
      }
      // Scale, mask (keys past S; causal keys after the query), tile max.
      float tmax = kNegInf;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = kt0 + 16 * mt + 4 * g + r;
          const bool ok = live[mt] && key < S && !(a.causal && key > qi);
          const float x = ok ? s[mt][r] * a.scale : kNegInf;
          s[mt][r] = x;
          tmax = fmaxf(tmax, x);
        }
      }
      tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
      const float m_new = fmaxf(m, tmax);
      // A row with every key so far masked keeps m = -inf (exp(-inf - -inf) would be NaN).
      const bool none = m_new == kNegInf;
      const float alpha = none ? 1.0f : exp2_hw((m - m_new) * kLog2e);
      float psum = 0.0f;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = none ? 0.0f : exp2_hw((s[mt][r] - m_new) * kLog2e);
          s[mt][r] = p;
          psum += p;
        }
      }
      lsum = lsum * alpha + psum;
      m = m_new;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) acc[mt] *= alpha;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        if (!live[kt]) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float* vr = Vt + (16 * kt + 4 * g + r) * kFwdLd + lo;
          const float p = s[kt][r];
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) acc[mt] = mma(vr[16 * mt], p, acc[mt]);
        }
      }
    }
    if (has_next) sstore(buf ^ 1);  // that buffer's last readers passed the previous barrier
    __syncthreads();
  }

  if (wave_live) {
    // The row sum: the four lanes of a query hold partial sums over disjoint keys; every lane
    // adds them in the same order.
    const float l0 = __shfl(lsum, lo), l1 = __shfl(lsum, lo + 16);
    const float l2 = __shfl(lsum, lo + 32), l3 = __shfl(lsum, lo + 48);
    const float l = (l0 + l1) + (l2 + l3);
    if (qi < S) {
      const float inv = 1.0f / l;
      float* orow = a.o + ((static_cast<int64_t>(b) * S + qi) * a.H + h) * kHeadDim;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) st4(orow + 16 * mt + 4 * g, acc[mt] * inv);
      if (g == 0) a.lse[static_cast<int64_t>(bh) * S + qi] = m + logf(l);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Backward, step 1: D[b, h, i] = sum_c dO[b, i, h, c] O[b, i, h, c]. 16 lanes per row (one float4
// each, then the xor butterfly 8, 4, 2, 1: one fixed order). It also clears the turn counters,
// the ticket and the guard word of step 2 (stream order puts it first).
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(kThreads) prep_kernel(const float* __restrict__ o, View d_o,
                                                       float* __restrict__ dsum,
                                                       int* __restrict__ turn,
                                                       int* __restrict__ ctrl, int B, int H,
                                                       int S, int nturn) {
  const int gtid = static_cast<int>(blockIdx.x) * kThreads + static_cast<int>(threadIdx.x);
  if (gtid < nturn) turn[gtid] = 0;
  if (gtid < 64) ctrl[gtid] = 0;
  const int64_t rows = static_cast<int64_t>(B) * H * S;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x >> 4);
  const int c4 = threadIdx.x & 15;
  float x = 0.0f;
  if (row < rows) {
    const int i = static_cast<int>(row % S);
    const int64_t bh = row / S;
    const int h = static_cast<int>(bh % H), b = static_cast<int>(bh / H);
    const f4 ov = ld4(o + ((static_cast<int64_t>(b) * S + i) * H + h) * kHeadDim + 4 * c4);
    const f4 gv = ld4(d_o.p + b * d_o.sb + h * d_o.sh + i * d_o.ss + 4 * c4);
    x = ov.x * gv.x;
    x = fmaf(ov.y, gv.y, x);
    x = fmaf(ov.z, gv.z, x);
    x = fmaf(ov.w, gv.w, x);
  }
  x += __shfl_xor(x, 8);
  x += __shfl_xor(x, 4);
  x += __shfl_xor(x, 2);
  x += __shfl_xor(x, 1);
  if (row < rows && c4 == 0) dsum[row] = x;
}

// ---------------------------------------------------------------------------------------------
// Backward, step 2. One workgroup = one key block of 64 keys of one (b, h); wave w owns keys
// k0 + 16 w .. + 15, one per lane column lo, with K and V of its key in registers (the B operands)
// and dK^T, dV^T of its keys in accumulators. It walks query tiles of 16 (causal: from the block's
// first key on), the next tile's Q, dO, L, D in flight during this one (double buffer).
//   S = Q K^T and dP = dO V^T: M = queries, N = the wave's keys, contraction over d;
//   A = Q / dO [query lo][dim 16 g + t] (LDS), B = K / V [key lo][dim 16 g + t] (registers).
//   P = exp(S scale - L), dS = P o (dP - D), in place in the accumulators.
//   dV^T += dO^T P, dK^T += Q^T dS: M = dims, N = keys, contraction over the tile's queries;
//   step r uses query 4 g + r, i.e. the P / dS value lane (lo, g) holds in register r.
//   dQ partial = dS K over the block's 64 keys: dS goes through LDS (the only product that needs
//   the queries in lo); wave w computes dims 16 w .. + 15, step t contracting keys 4 t + g.
// The partial is added into dQ on the tile's turn: key block 0 stores, the others read, add and
// store, the last contributor scales; then the turn passes to the next key block. The tile's dQ
// is therefore ((p0 + p1) + p2) + ... in key-block order on every run.
// ---------------------------------------------------------------------------------------------
constexpr int kQT = kBwdQueryTile;  // 16
constexpr int kBwdLd = 68;          // Q / dO / dS tile pitch (floats)
constexpr int kBwdKLd = 80;         // K block pitch: conflict-free reads of K[4 t + g][16 w + lo]

struct BwdArgs {
  View q, k, v, d_o;
  const float* lse;
  const float* dsum;
  float* dqkv;
  int* turn;
  int* ctrl;
  int B, H, S, nkb, ntile;
  float scale;
  int causal;
};

// The dQ hand-over between key blocks. MI355X has one L2 per XCD and the L2s are not coherent
// with each other, so an agent-scope release / acquire fence pair has to write back / invalidate
// a whole L2 -- per tile, per workgroup, far more than the 16 x 64 floats that change hands. The
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
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Spin until the turn counter reads `want`. Bounded: on timeout the guard word is raised.
__device__ __forceinline__ void wait_turn(int* p, int want, int* guard) {
  int spins = 0;
  while (__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != want) {
    __builtin_amdgcn_s_sleep(2);
    ++spins;
    // Once any wait of this launch has timed out, the others stop waiting too.
    if (spins > kSpinBound ||
        ((spins & 63) == 0 &&
         __hip_atomic_load(guard, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0)) {
      __hip_atomic_store(guard, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
  }
}

__global__ void __launch_bounds__(kThreads) bwd_kernel(BwdArgs a) {
  __shared__ __attribute__((aligned(16))) float sQ[2][kQT * kBwdLd];
  __shared__ __attribute__((aligned(16))) float sdO[2][kQT * kBwdLd];
  __shared__ __attribute__((aligned(16))) float sdS[kQT * kBwdLd];
  __shared__ __attribute__((aligned(16))) float sK[kBwdKeys * kBwdKLd];
  __shared__ float sL[2][kQT], sD[2][kQT];
  __shared__ int s_item;

  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, lo = lane & 15, g = lane >> 4;
  // Ticket: the key block this workgroup computes, in arrival order. Key block kb of a (b, h) is
  // item bh * nkb + kb, so the block it waits on (kb - 1) was taken by an earlier, running one.
  if (tid == 0) s_item = atomicAdd(a.ctrl + kCtrlTicket, 1);
  __syncthreads();
  const int item = s_item;
  if (item >= a.nkb * a.B * a.H) {
    // The ticket was not cleared by step 1 on this workspace: refuse (no access out of range),
    // and raise the guard word so the caller can tell.
    if (tid == 0) __hip_atomic_store(a.ctrl + kCtrlGuard, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  const int bh = item / a.nkb, kb = item % a.nkb;
  const int b = bh / a.H, h = bh % a.H, S = a.S;
  const int k0 = kb * kBwdKeys;
  const int kw0 = k0 + 16 * w;  // the wave's first key
  const int key = kw0 + lo;     // this lane's key

  const float* qp = a.q.p + b * a.q.sb + h * a.q.sh;
  const float* kp = a.k.p + b * a.k.sb + h * a.k.sh;
  const float* vp = a.v.p + b * a.v.sb + h * a.v.sh;
  const float* gp = a.d_o.p + b * a.d_o.sb + h * a.d_o.sh;
  const float* lp = a.lse + static_cast<int64_t>(bh) * S;
  const float* dp = a.dsum + static_cast<int64_t>(bh) * S;
  int* tp = a.turn + static_cast<int64_t>(bh) * a.ntile;

  // B operands of S and dP: K[key][16 g .. 16 g + 15], V likewise.
  float kB[16], vB[16];
  if (key < S) {
    const float* kr = kp + key * a.k.ss + 16 * g;
    const float* vr = vp + key * a.v.ss + 16 * g;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const f4 x = ld4(kr + 4 * u), y = ld4(vr + 4 * u);
      kB[4 * u] = x.x;
      kB[4 * u + 1] = x.y;
      kB[4 * u + 2] = x.z;
      kB[4 * u + 3] = x.w;
      vB[4 * u] = y.x;
      vB[4 * u + 1] = y.y;
      vB[4 * u + 2] = y.z;
      vB[4 * u + 3] = y.w;
    }
  } else {
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      kB[t] = 0.0f;
      vB[t] = 0.0f;
    }
  }
  // The key block's K, for the dQ product; zero rows past S.
  const int srow = tid >> 4, sc4 = tid & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = srow + 16 * i, kk = k0 + row;
    const f4 x = kk < S ? ld4(kp + kk * a.k.ss + 4 * sc4) : zero4();
    st4(&sK[row * kBwdKLd + 4 * sc4], x);
  }

  // Staging of one query tile: thread tid moves Q and dO row tid / 16, float4 column tid % 16;
  // threads 0..15 move L, 16..31 move D. Zero past S.
  f4 qst = zero4(), gst = zero4();
  float lst = 0.0f;
  auto gload = [&](int q0) {
    const int qq = q0 + srow;
    if (qq < S) {
      qst = ld4(qp + qq * a.q.ss + 4 * sc4);
      gst = ld4(gp + qq * a.d_o.ss + 4 * sc4);
    } else {
      qst = zero4();
      gst = zero4();
    }
    if (tid < 16) {
      lst = q0 + tid < S ? lp[q0 + tid] : 0.0f;
    } else if (tid < 32) {
      lst = q0 + tid - 16 < S ? dp[q0 + tid - 16] : 0.0f;
    }
  };
  auto sstore = [&](int buf) {
    st4(&sQ[buf][srow * kBwdLd + 4 * sc4], qst);
    st4(&sdO[buf][srow * kBwdLd + 4 * sc4], gst);
    if (tid < 16) {
      sL[buf][tid] = lst;
    } else if (tid < 32) {
      sD[buf][tid - 16] = lst;
    }
  };

  f4 dva[4], dka[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    dva[mt] = zero4();
    dka[mt] = zero4();
  }

  // Causal: queries before the block's first key see none of its keys.
  const int q_begin = a.causal ? k0 : 0;
  gload(q_begin);
  sstore(0);
  __syncthreads();
  for (int t = 0, q0 = q_begin; q0 < S; ++t, q0 += kQT) {
    const int buf = t & 1;
    const bool has_next = q0 + kQT < S;
    if (has_next) gload(q0 + kQT);
    const float* Qt = sQ[buf];
    const float* Gt = sdO[buf];
    // Wave-uniform liveness of each wave's 16 keys for this tile (all masked: skip the math).
    int live_mask = 0;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      const int kx = k0 + 16 * ww;
      if (kx < S && !(a.causal && kx > q0 + kQT - 1)) live_mask |= 1 << ww;
    }

    f4 dS = zero4();
    if (live_mask & (1 << w)) {
      f4 sS = zero4(), sP = zero4();
      const float* qr = Qt + lo * kBwdLd + 16 * g;
      const float* gr = Gt + lo * kBwdLd + 16 * g;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const f4 x = ld4(qr + 4 * u), y = ld4(gr + 4 * u);
        sS = mma(x.x, kB[4 * u], sS);
        sS = mma(x.y, kB[4 * u + 1], sS);
        sS = mma(x.z, kB[4 * u + 2], sS);
        sS = mma(x.w, kB[4 * u + 3], sS);
        sP = mma(y.x, vB[4 * u], sP);
        sP = mma(y.y, vB[4 * u + 1], sP);
        sP = mma(y.z, vB[4 * u + 2], sP);
        sP = mma(y.w, vB[4 * u + 3], sP);
      }
      // Lane (lo, g), register r: query q0 + 4 g + r, key `key`.
      f4 P;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int il = 4 * g + r, qi = q0 + il;
        const bool ok = qi < S && key < S && !(a.causal && key > qi);
        P[r] = ok ? exp2_hw(fmaf(sS[r], a.scale, -sL[buf][il]) * kLog2e) : 0.0f;
        dS[r] = P[r] * (sP[r] - sD[buf][il]);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float* grow = Gt + (4 * g + r) * kBwdLd + lo;
        const float* qrow = Qt + (4 * g + r) * kBwdLd + lo;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          dva[mt] = mma(grow[16 * mt], P[r], dva[mt]);
          dka[mt] = mma(qrow[16 * mt], dS[r], dka[mt]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) sdS[(4 * g + r) * kBwdLd + 16 * w + lo] = dS[r];
    __syncthreads();

    // dQ partial for dims 16 w + lo; step t4 contracts keys 4 t4 + g (keys of wave t4 / 4).
    f4 dq = zero4();
#pragma unroll
    for (int t4 = 0; t4 < 16; ++t4) {
      if (!(live_mask & (1 << (t4 >> 2)))) continue;
      const int kl = 4 * t4 + g;
      dq = mma(sdS[lo * kBwdLd + kl], sK[kl * kBwdKLd + 16 * w + lo], dq);
    }
    if (has_next) sstore(buf ^ 1);  // that buffer's last readers passed the previous barrier

    // Ordered accumulation of the tile's dQ over key blocks 0 .. last.
    const int tile = q0 / kQT;
    const int last =
        a.causal ? min(a.nkb - 1, min(S - 1, q0 + kQT - 1) / kBwdKeys) : a.nkb - 1;
    if (kb > 0) {
      if (tid == 0) wait_turn(tp + tile, kb, a.ctrl + kCtrlGuard);
      __syncthreads();  // no wave reads dQ before the turn is seen
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int qi = q0 + 4 * g + r;
      if (qi < S) {
        float* dst = a.dqkv + ((static_cast<int64_t>(b) * S + qi) * 3 * a.H + h) * kHeadDim +
                     16 * w + lo;
        float x = dq[r];
        if (kb > 0) x = ld_agent(dst) + x;
        if (kb == last) x *= a.scale;
        st_agent(dst, x);
      }
    }
    if (kb < last) {
      wait_stores();    // this wave's dQ stores are complete at the coherence point
      __syncthreads();  // ... and every other wave's
      if (tid == 0) __hip_atomic_store(tp + tile, kb + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if (kb == 0) {
      __syncthreads();  // no other barrier this iteration: dS and the staging buffer are reused
    }
  }

  // dK (x scale) and dV of this lane's key: dims 16 mt + 4 g .. + 3, one float4 each.
  if (key < S) {
    float* row = a.dqkv + (static_cast<int64_t>(b) * S + key) * 3 * a.H * kHeadDim +
                 static_cast<int64_t>(h) * kHeadDim;
    const int64_t part = static_cast<int64_t>(a.H) * kHeadDim;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      st4(row + part + 16 * mt + 4 * g, dka[mt] * a.scale);
      st4(row + 2 * part + 16 * mt + 4 * g, dva[mt]);
    }
  }
}

}  // namespace

int64_t forward_blocks(int64_t b, int64_t h, int64_t s) {
  return ((s + kFwdQueries - 1) / kFwdQueries) * h * b;
}
int64_t bwd_main_blocks(int64_t b, int64_t h, int64_t s) {
  return ((s + kBwdKeys - 1) / kBwdKeys) * h * b;
}
int64_t bwd_prep_blocks(int64_t b, int64_t h, int64_t s) { return (b * h * s + 15) / 16; }

int launch_forward(View q, View k, View v, float* o, float* lse, int b, int h, int s,
                   float scale, int causal, void* stream) {
  FwdArgs a{q, k, v, o, lse, b, h, s, (s + kFwdQueries - 1) / kFwdQueries, scale, causal};
  void* args[] = {&a};
  return static_cast<int>(hipLaunchKernel(reinterpret_cast<const void*>(fwd_kernel),
                                          dim3(static_cast<unsigned>(forward_blocks(b, h, s))),
                                          dim3(kThreads), args, 0,
                                          static_cast<hipStream_t>(stream)));
}

int launch_bwd_prep(const float* o, View d_o, float* dsum, int* turn, int* ctrl, int b, int h,
                    int s, void* stream) {
  int nturn = b * h * ((s + kQT - 1) / kQT);
  void* args[] = {&o, &d_o, &dsum, &turn, &ctrl, &b, &h, &s, &nturn};
  return static_cast<int>(hipLaunchKernel(reinterpret_cast<const void*>(prep_kernel),
                                          dim3(static_cast<unsigned>(bwd_prep_blocks(b, h, s))),
                                          dim3(kThreads), args, 0,
                                          static_cast<hipStream_t>(stream)));
}

int launch_bwd_main(View q, View k, View v, View d_o, const float* lse, const float* dsum,
                    float* dqkv, int* turn, int* ctrl, int b, int h, int s, float scale,
                    int causal, void* stream) {
  BwdArgs a{q, k, v, d_o, lse, dsum, dqkv, turn, ctrl, b, h, s,
            (s + kBwdKeys - 1) / kBwdKeys, (s + kQT - 1) / kQT, scale, causal};
  void* args[] = {&a};
  return static_cast<int>(hipLaunchKernel(reinterpret_cast<const void*>(bwd_kernel),
                                          dim3(static_cast<unsigned>(bwd_main_blocks(b, h, s))),
                                          dim3(kThreads), args, 0,
                                          static_cast<hipStream_t>(stream)));
}

}  // namespace fattn
