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

/* S[i][j] = (q_i . k_j), summed over c in index order (the slice functions' order). */
static REAL FN(dot_)(const REAL* a, const REAL* b, int64_t d) {
  REAL acc = 0;
  for (int64_t c = 0; c < d; ++c) acc += a[c] * b[c];
  return acc;
}

/* One (batch, head) slice at sampled rows, for sequences whose [s][s] scores the slice
 * functions above cannot hold: O and L at query rows rows[0..nr), dQ at the same rows, dK and
 * dV at key rows keys[0..nk). The formulas and the order of every sum are those of fwd_slice_
 * and bwd_slice_ (src/lib.rs:240-299), evaluated one row or column at a time, so the results
 * equal theirs bit for bit; O and L of every query row come first (the backward's
 * P = exp(S scale - L) and D = rowsum(dO o O) need them for every query), OpenMP-parallel over
 * rows, then dQ per sampled row and dK, dV per sampled key.
 * q, k, v, d_o contiguous [s][d]; outputs [nr][d], [nr], [nr][d], [nk][d], [nk][d].
 * Returns -1 on a bad argument or allocation failure. */
int FN(oracle_rows_)(const REAL* q, const REAL* k, const REAL* v, const REAL* d_o,
                    int64_t s, int64_t d, REAL scale, int causal, const int64_t* rows,
                    int64_t nr, const int64_t* keys, int64_t nk, REAL* o_rows,
                    REAL* l_rows, REAL* dq_rows, REAL* dk_keys, REAL* dv_keys,
                    int threads) {
  if (s <= 0 || d <= 0 || nr < 0 || nk < 0) return -1;
  for (int64_t r = 0; r < nr; ++r)
    if (rows[r] < 0 || rows[r] >= s) return -1;
  for (int64_t r = 0; r < nk; ++r)
    if (keys[r] < 0 || keys[r] >= s) return -1;
  REAL* o = (REAL*)malloc(sizeof(REAL) * (size_t)(s * d));
  REAL* l = (REAL*)malloc(sizeof(REAL) * (size_t)s);
  REAL* dsum = (REAL*)malloc(sizeof(REAL) * (size_t)s);
  if (!o || !l || !dsum) {
    free(o);
    free(l);
    free(dsum);
    return -1;
  }
  int bad = 0;
  const int nt = threads > 0 ? threads : 1;
  /* The forward of every query row (fwd_slice_), and D (bwd_slice_'s dsum). */
#pragma omp parallel num_threads(nt)
  {
    REAL* row = (REAL*)malloc(sizeof(REAL) * (size_t)s);
    if (!row) {
#pragma omp atomic write
      bad = 1;
    }
#pragma omp for schedule(dynamic, 16)
    for (int64_t i = 0; i < s; ++i) {
      if (!row) continue;
      REAL mx = -INFINITY;
      for (int64_t j = 0; j < s; ++j) {
        REAL t = FN(dot_)(q + i * d, k + j * d, d) * scale;
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
      REAL ds = 0;
      for (int64_t c = 0; c < d; ++c) ds += d_o[i * d + c] * orow[c];
      dsum[i] = ds;
    }
    free(row);
  }
  if (bad) {
    free(o);
    free(l);
    free(dsum);
    return -1;
  }
  /* dQ of the sampled query rows: sum over keys in index order, then times scale. */
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1)
  for (int64_t r = 0; r < nr; ++r) {
    const int64_t i = rows[r];
    REAL* dqi = dq_rows + r * d;
    for (int64_t c = 0; c < d; ++c) {
      o_rows[r * d + c] = o[i * d + c];
      dqi[c] = 0;
    }
    l_rows[r] = l[i];
    for (int64_t j = 0; j < s; ++j) {
      REAL pij = EXP(FN(dot_)(q + i * d, k + j * d, d) * scale - l[i]);
      if (causal && j > i) pij = 0;
      const REAL dsij = pij * (FN(dot_)(d_o + i * d, v + j * d, d) - dsum[i]);
      for (int64_t c = 0; c < d; ++c) dqi[c] += dsij * k[j * d + c];
    }
    for (int64_t c = 0; c < d; ++c) dqi[c] *= scale;
  }
  /* dK and dV of the sampled key rows: sums over queries in index order; dK times scale. */
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1)
  for (int64_t r = 0; r < nk; ++r) {
    const int64_t j = keys[r];
    REAL* dkj = dk_keys + r * d;
    REAL* dvj = dv_keys + r * d;
    for (int64_t c = 0; c < d; ++c) {
      dkj[c] = 0;
      dvj[c] = 0;
    }
    for (int64_t i = 0; i < s; ++i) {
      REAL pij = EXP(FN(dot_)(q + i * d, k + j * d, d) * scale - l[i]);
      if (causal && j > i) pij = 0;
      const REAL dsij = pij * (FN(dot_)(d_o + i * d, v + j * d, d) - dsum[i]);
      for (int64_t c = 0; c < d; ++c) {
        dvj[c] += pij * d_o[i * d + c];
        dkj[c] += dsij * q[i * d + c];
      }
    }
    for (int64_t c = 0; c < d; ++c) dkj[c] *= scale;
  }
  free(o);
  free(l);
  free(dsum);
  return 0;
}

#undef FN
#undef CAT
#undef CAT2
