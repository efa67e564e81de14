/*
 * oracle/composed.c -- TEST INFRASTRUCTURE, NOT THE PRODUCT.
 *
 * A CPU restatement, in plain C, of the reference crate's composed attention path
 * (mi-for-the-rust-of-us/candle-fused-attn v0.4.0, src/lib.rs):
 *   - oracle_gather_f32     = gather_cpu            (src/lib.rs:222-238)
 *   - oracle_forward_f32    = composed_forward      (src/lib.rs:240-259) + causal_bias (:261-267)
 *   - oracle_backward_f32   = composed_backward     (src/lib.rs:269-299)
 *   - oracle_forward_f64 / oracle_backward_f64: the same formulas in double precision, the
 *     fp64 recompute every result is scored against (bench/compare.py:506-536 scores against
 *     torch fp64 autograd of the same composition);
 *   - oracle_rows_f32 / oracle_rows_f64: the same, at sampled rows of one slice, for sequences
 *     too long for [s][s] buffers (bit-identical to the rows of the functions above).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this library, and
 * only as the checker or the timed CPU baseline -- never as a path of the shipped operator.
 *
 * Parity of this restatement is pinned (tests/test_oracle.py) by: torch float64 autograd of an
 * independently written composed attention (tests/golden/), central finite differences of the
 * forward (gradients), the closed forms of special cases (q = 0 -> uniform attention, s = 1,
 * equal value rows) and the gradient invariants (sum_j dK_j = 0, sum_j dV_j = sum_i dO_i).
 * The fp32 instance is NOT bit-identical to candle's CPU matmul (gemm crate), which is absent:
 * bit parity at that boundary is unpinned; only tolerance parity is claimed.
 *
 * Layout: q, k, v, o, dO, dq, dk, dv contiguous [b][h][s][d]; L [b][h][s].
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

/* float instance: the reference's fp32 CPU path */
#define REAL float
#define SUFFIX f32
#define EXP expf
#define LOG logf
#include "composed_impl.h"
#undef REAL
#undef SUFFIX
#undef EXP
#undef LOG

/* double instance: the fp64 recompute */
#define REAL double
#define SUFFIX f64
#define EXP exp
#define LOG log
#include "composed_impl.h"
#undef REAL
#undef SUFFIX
#undef EXP
#undef LOG

/* gather_cpu (src/lib.rs:222-238): a strided [b, h, s, d] operand of a flat f32 storage into a
 * contiguous buffer. Returns -1 if any element lies outside the storage (the reference's
 * "layout outside its storage" error), 0 otherwise. */
int oracle_gather_f32(const float* storage, int64_t storage_len, int64_t start, int64_t b,
                      int64_t h, int64_t s, int64_t d, int64_t sb, int64_t sh, int64_t ss,
                      float* dst) {
  int64_t e = 0;
  for (int64_t bi = 0; bi < b; ++bi)
    for (int64_t hi = 0; hi < h; ++hi)
      for (int64_t si = 0; si < s; ++si)
        for (int64_t di = 0; di < d; ++di) {
          const int64_t idx = start + bi * sb + hi * sh + si * ss + di;
          if (idx < 0 || idx >= storage_len) return -1;
          dst[e++] = storage[idx];
        }
  return 0;
}

const char* oracle_version(void) { return "composed-oracle 1 (src/lib.rs:222-299 restated)"; }
