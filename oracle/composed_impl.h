/*
 * Body of the composed attention, instantiated twice by composed.c: REAL = float (the
 * reference's CPU path restated in fp32) and REAL = double (the fp64 recompute the GPU results
 * are scored against). TEST INFRASTRUCTURE ONLY -- see composed.c.
 *
 * Operands of one (batch, head) slice are contiguous [s][d]; a call walks all b*h slices,
 * OpenMP-parallel over slices.
 */
#ifndef REAL
#error "define REAL and SUFFIX before including composed_impl.h"
#endif

#define CAT2(a, b) a##b
#define CAT(a, b) CAT2(a, b)
#define FN(name) CAT(name, SUFFIX)

/* Forward of one slice (src/lib.rs:241-259, composed_forward):
 *   scores = (q k^T) * scale            (src/lib.rs:248)
 *   causal: scores + (-inf where j > i)  (src/lib.rs:249-253, causal_bias :262-267)
 *   max = rowmax(scores); e = exp(scores - max); sum = rowsum(e)   (:254-256)
 *   o = (e / sum) v                      (:257)
 *   L = max + log(sum)                   (:258)
 * Work buffers: sc [s][s], kt [d][s]. */
static void FN(fwd_slice_)(const REAL* q, const REAL* k, const REAL* v, int64_t s, int64_t d,
                           REAL scale, int causal, REAL* o, REAL* l, REAL* sc, REAL* kt) {
  for (int64_t j = 0; j < s; ++j)
    for (int64_t c = 0; c < d; ++c) kt[c * s + j] = k[j * d + c];
  for (int64_t i = 0; i < s; ++i) {
    REAL* row = sc + i * s;
    for (int64_t j = 0; j < s; ++j) row[j] = 0;
    /* row[j] = sum_c q[i][c] k[j][c], summed over c in index order */
    for (int64_t c = 0; c < d; ++c) {
      const REAL x = q[i * d + c];
      const REAL* kr = kt + c * s;
      for (int64_t j = 0; j < s; ++j) row[j] += x * kr[j];
    }
    REAL mx = -INFINITY;
    for (int64_t j = 0; j < s; ++j) {
      REAL t = row[j] * scale;
      if (causal && j > i) t = -INFINITY;
      row[j] = t;
      if (t > mx) mx = t;
    }
    REAL sum = 0;
    for (int64_t j = 0; j < s; ++j) {
      row[j] = EXP(row[j] - mx);
      sum += row[j];
    }
    REAL* orow = o + i * d;
    for (int64_t c = 0; c < d; ++c) orow[c] = 0;
    for (int64_t j = 0; j < s; ++j) {
      const REAL p = row[j] / sum;
      const REAL* vr = v + j * d;
      for (int64_t c = 0; c < d; ++c) orow[c] += p * vr[c];
    }
    l[i] = mx + LOG(sum);
  }
}

/* Backward of one slice (src/lib.rs:269-299, composed_backward), P recomputed from L:
 *   p  = exp((q k^T) * scale - L)  (x keep = exp(causal_bias): 1 where j <= i, 0 above)
 *   dv = p^T dO ;  dp = dO v^T ;  D = rowsum(dO o O) ;  ds = p o (dp - D)
 *   dq = (ds k) * scale ;  dk = (ds^T q) * scale
 * Work buffers: p [s][s], dp [s][s], kt [d][s], vt [d][s]. */
static void FN(bwd_slice_)(const REAL* q, const REAL* k, const REAL* v, const REAL* o,
                           const REAL* l, const REAL* d_o, int64_t s, int64_t d, REAL scale,
                           int causal, REAL* dq, REAL* dk, REAL* dv, REAL* p, REAL* dp, REAL* kt,
                           REAL* vt) {
  for (int64_t j = 0; j < s; ++j)
    for (int64_t c = 0; c < d; ++c) {
      kt[c * s + j] = k[j * d + c];
      vt[c * s + j] = v[j * d + c];
    }
  for (int64_t i = 0; i < s; ++i) {
    REAL* prow = p + i * s;
    REAL* dprow = dp + i * s;
    for (int64_t j = 0; j < s; ++j) {
      prow[j] = 0;
      dprow[j] = 0;
    }
    for (int64_t c = 0; c < d; ++c) {
      const REAL x = q[i * d + c], y = d_o[i * d + c];
      const REAL* kr = kt + c * s;
      const REAL* vr = vt + c * s;
      for (int64_t j = 0; j < s; ++j) {
        prow[j] += x * kr[j];
        dprow[j] += y * vr[j];
      }
    }
    REAL dsum = 0;
    for (int64_t c = 0; c < d; ++c) dsum += d_o[i * d + c] * o[i * d + c];
    for (int64_t j = 0; j < s; ++j) {
      REAL pij = EXP(prow[j] * scale - l[i]);
      if (causal && j > i) pij = 0;
      prow[j] = pij;
      dprow[j] = pij * (dprow[j] - dsum); /* ds */
    }
  }
  for (int64_t x = 0; x < s * d; ++x) {
    dq[x] = 0;
    dk[x] = 0;
    dv[x] = 0;
  }
  for (int64_t i = 0; i < s; ++i) {
    const REAL* prow = p + i * s;
    const REAL* dsrow = dp + i * s;
    const REAL* gi = d_o + i * d;
    const REAL* qi = q + i * d;
    REAL* dqi = dq + i * d;
    for (int64_t j = 0; j < s; ++j) {
      const REAL pij = prow[j], dsij = dsrow[j];
      REAL* dvj = dv + j * d;
      REAL* dkj = dk + j * d;
      const REAL* kj = k + j * d;
      for (int64_t c = 0; c < d; ++c) {
        dvj[c] += pij * gi[c];
        dkj[c] += dsij * qi[c];
        dqi[c] += dsij * kj[c];
      }
    }
  }
  for (int64_t x = 0; x < s * d; ++x) {
    dq[x] *= scale;
    dk[x] *= scale;
  }
}

int FN(oracle_forward_)(const REAL* q, const REAL* k, const REAL* v, int64_t b, int64_t h,
                        int64_t s, int64_t d, REAL scale, int causal, REAL* o, REAL* l,
                        int threads) {
  if (b < 0 || h < 0 || s < 0 || d < 0) return -1;
  const int64_t n = b * h;
  if (n == 0 || s == 0) return 0;
  int bad = 0;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
  {
    REAL* sc = (REAL*)malloc(sizeof(REAL) * (size_t)(s * s + d * s));
    if (!sc) {
#pragma omp atomic write
      bad = 1;
    } else {
#pragma omp for schedule(dynamic, 1)
      for (int64_t x = 0; x < n; ++x) {
        const int64_t off = x * s * d;
        FN(fwd_slice_)(q + off, k + off, v + off, s, d, scale, causal, o + off, l + x * s, sc,
                       sc + s * s);
      }
      free(sc);
    }
  }
  return bad ? -2 : 0;
}

int FN(oracle_backward_)(const REAL* q, const REAL* k, const REAL* v, const REAL* o,
                         const REAL* l, const REAL* d_o, int64_t b, int64_t h, int64_t s,
                         int64_t d, REAL scale, int causal, REAL* dq, REAL* dk, REAL* dv,
                         int threads) {
  if (b < 0 || h < 0 || s < 0 || d < 0) return -1;
  const int64_t n = b * h;
  if (n == 0 || s == 0) return 0;
  int bad = 0;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
  {
    REAL* w = (REAL*)malloc(sizeof(REAL) * (size_t)(2 * s * s + 2 * d * s));
    if (!w) {
#pragma omp atomic write
      bad = 1;
    } else {
#pragma omp for schedule(dynamic, 1)
      for (int64_t x = 0; x < n; ++x) {
        const int64_t off = x * s * d;
        FN(bwd_slice_)(q + off, k + off, v + off, o + off, l + x * s, d_o + off, s, d, scale,
                       causal, dq + off, dk + off, dv + off, w, w + s * s, w + 2 * s * s,
                       w + 2 * s * s + d * s);
      }
      free(w);
    }
  }
  return bad ? -2 : 0;
}

#undef FN
#undef CAT
#undef CAT2
