/*
 * spconv_oracle.c -- CPU restatement of the spconv-Triton sparse-convolution
 * hot path.  TEST INFRASTRUCTURE ONLY: this file is the checker that the HIP
 * library is compared against (tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py).  The product path never links or calls it.
 *
 * It deliberately follows the reference's own algorithm (sort + lower-bound
 * membership, torch.unique for output keys, per-offset compaction), not the
 * hash / bitmap design of the GPU library, so that agreement between the two
 * is evidence rather than a tautology.
 *
 * Reference files followed (paths relative to the reference repository):
 *   spconv_triton/pytorch/_impl/pairs.py        (whole file)
 *   spconv_triton/pytorch/_impl/pair_kernels.py :37-94, :159-183, :220-261,
 *                                               :298-358, :398-446
 *   spconv_triton/pytorch/_impl/gemm.py         :254-321 (fwd/dgrad), :356-426 (wgrad)
 *   spconv_triton/pytorch/_impl/pool.py         :45-257
 *
 * Keys are always int64 here.  The reference picks int32 keys when
 * batch*volume < 2^31 (pairs.py:166-171); valid keys are identical in both
 * widths (pair_kernels.py:12-16), so int64 reproduces every consumed value.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* stable sort helpers: merge sort of (key, index) pairs, ties by index.     */
/* ------------------------------------------------------------------------ */
typedef struct { int64_t key; int64_t idx; } kv_pair;

static void merge_sort_pairs(kv_pair* a, kv_pair* tmp, int64_t n) {
  /* bottom-up, stable */
  for (int64_t width = 1; width < n; width *= 2) {
    for (int64_t lo = 0; lo < n; lo += 2 * width) {
      int64_t mid = lo + width < n ? lo + width : n;
      int64_t hi = lo + 2 * width < n ? lo + 2 * width : n;
      int64_t i = lo, j = mid, o = lo;
      while (i < mid && j < hi) {
        if (a[j].key < a[i].key) tmp[o++] = a[j++];
        else tmp[o++] = a[i++];
      }
      while (i < mid) tmp[o++] = a[i++];
      while (j < hi) tmp[o++] = a[j++];
    }
    memcpy(a, tmp, (size_t)n * sizeof(kv_pair));
  }
}

/* ------------------------------------------------------------------------ */
/* kernel offsets: row-major, last dim fastest (pairs.py:43-48)              */
/* ------------------------------------------------------------------------ */
int orc_kernel_offsets(int ndim, const int64_t* ksize, int64_t* offs) {
  int64_t kv = 1;
  for (int d = 0; d < ndim; ++d) kv *= ksize[d];
  for (int64_t k = 0; k < kv; ++k) {
    int64_t rem = k;
    for (int d = ndim - 1; d >= 0; --d) {
      offs[k * ndim + d] = rem % ksize[d];
      rem /= ksize[d];
    }
  }
  return 0;
}

/* floor division for int64 (torch // on the numerator; only o>=0 survives) */
static int64_t floordiv(int64_t a, int64_t b) {
  int64_t q = a / b;
  if ((a % b != 0) && ((a < 0) != (b < 0))) q -= 1;
  return q;
}

/* ------------------------------------------------------------------------ */
/* candidate out key + geometric validity (pair_kernels.py:57-94)            */
/* lane off = k*N + j                                                        */
/* ------------------------------------------------------------------------ */
int orc_candidates(const int32_t* idx, int64_t N, int ndim, const int64_t* ksize,
                   const int64_t* pad, const int64_t* stride, const int64_t* dil,
                   const int64_t* out_shape, int transpose, int strided,
                   int64_t* out_lin, uint8_t* valid) {
  int64_t kv = 1;
  for (int d = 0; d < ndim; ++d) kv *= ksize[d];
  int64_t* offs = (int64_t*)malloc(sizeof(int64_t) * (size_t)(kv * ndim));
  orc_kernel_offsets(ndim, ksize, offs);
  const int W = ndim + 1;
#pragma omp parallel for schedule(static)
  for (int64_t k = 0; k < kv; ++k) {
    for (int64_t j = 0; j < N; ++j) {
      int64_t acc = idx[j * W];
      int ok = 1;
      for (int d = 0; d < ndim; ++d) {
        int64_t c = idx[j * W + d + 1];
        int64_t off = offs[k * ndim + d] * dil[d];
        int64_t osh = out_shape[d];
        int64_t contrib;
        if (transpose) {
          int64_t o = c * stride[d] + off - pad[d];
          ok = ok && (o >= 0) && (o < osh);
          contrib = o;
        } else {
          int64_t o = c + pad[d] - off;
          if (strided) {
            int64_t q = floordiv(o, stride[d]);
            ok = ok && (o >= 0) && (o - q * stride[d] == 0) && (q < osh);
            contrib = q;
          } else {
            ok = ok && (o >= 0) && (o < osh);
            contrib = o;
          }
        }
        acc = acc * osh + contrib;
      }
      out_lin[k * N + j] = acc;
      valid[k * N + j] = (uint8_t)ok;
    }
  }
  free(offs);
  return 0;
}

/* batch-major linear key of every input row (pairs.py:91-95) */
int orc_linearize(const int32_t* idx, int64_t N, int ndim, const int64_t* shape,
                  int64_t* lin) {
  const int W = ndim + 1;
  for (int64_t j = 0; j < N; ++j) {
    int64_t acc = idx[j * W];
    for (int d = 0; d < ndim; ++d) acc = acc * shape[d] + idx[j * W + d + 1];
    lin[j] = acc;
  }
  return 0;
}

/* lower bound in a sorted int64 array */
static int64_t lower_bound64(const int64_t* s, int64_t n, int64_t t) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    int64_t mid = (lo + hi) / 2;
    if (s[mid] < t) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

/* ------------------------------------------------------------------------ */
/* subm membership: sort input keys, lower-bound each candidate              */
/* (pairs.py:196-204, pair_kernels.py:420-446)                               */
/* valid is updated in place (prior AND found); out_row gets the input row   */
/* ------------------------------------------------------------------------ */
int orc_subm_membership(const int64_t* out_lin, uint8_t* valid, int64_t kv, int64_t N,
                        const int64_t* in_lin, int32_t* out_row) {
  kv_pair* a = (kv_pair*)malloc(sizeof(kv_pair) * (size_t)N);
  kv_pair* t = (kv_pair*)malloc(sizeof(kv_pair) * (size_t)N);
  int64_t* sorted = (int64_t*)malloc(sizeof(int64_t) * (size_t)N);
  for (int64_t j = 0; j < N; ++j) { a[j].key = in_lin[j]; a[j].idx = j; }
  merge_sort_pairs(a, t, N);
  for (int64_t j = 0; j < N; ++j) sorted[j] = a[j].key;
#pragma omp parallel for schedule(static)
  for (int64_t off = 0; off < kv * N; ++off) {
    int64_t target = out_lin[off];
    int64_t pos = lower_bound64(sorted, N, target);
    int found = (pos < N) && (sorted[pos] == target);
    int64_t pc = pos < N ? pos : N - 1;
    out_row[off] = (int32_t)a[pc].idx;
    valid[off] = (uint8_t)(valid[off] && found);
  }
  free(a); free(t); free(sorted);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* regular/transpose: sorted unique valid keys (torch.unique, pairs.py:206)  */
/* returns n_out; uniq must hold kv*N entries                                */
/* ------------------------------------------------------------------------ */
int64_t orc_unique_sorted(const int64_t* out_lin, const uint8_t* valid, int64_t n,
                          int64_t* uniq) {
  int64_t m = 0;
  for (int64_t i = 0; i < n; ++i) if (valid[i]) ++m;
  if (m == 0) return 0;
  kv_pair* a = (kv_pair*)malloc(sizeof(kv_pair) * (size_t)m);
  kv_pair* t = (kv_pair*)malloc(sizeof(kv_pair) * (size_t)m);
  int64_t p = 0;
  for (int64_t i = 0; i < n; ++i) if (valid[i]) { a[p].key = out_lin[i]; a[p].idx = i; ++p; }
  merge_sort_pairs(a, t, m);
  int64_t u = 0;
  for (int64_t i = 0; i < m; ++i) {
    if (i == 0 || a[i].key != a[i - 1].key) uniq[u++] = a[i].key;
  }
  free(a); free(t);
  return u;
}

/* out_row = lower-bound position in uniq for valid lanes, 0 otherwise
   (pair_kernels.py:349-358) */
int orc_lower_bound_rows(const int64_t* out_lin, const uint8_t* valid, int64_t n,
                         const int64_t* uniq, int64_t n_out, int32_t* out_row) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    out_row[i] = valid[i] ? (int32_t)lower_bound64(uniq, n_out, out_lin[i]) : 0;
  }
  return 0;
}

/* keys -> [n, ndim+1] int32 coordinates (pairs.py:98-111) */
int orc_delinearize(const int64_t* lin, int64_t n, int ndim, const int64_t* shape,
                    int32_t* out) {
  const int W = ndim + 1;
  for (int64_t i = 0; i < n; ++i) {
    int64_t rem = lin[i];
    for (int d = ndim - 1; d >= 0; --d) {
      /* torch % and // are floor ops; keys are non-negative here */
      out[i * W + d + 1] = (int32_t)(rem % shape[d]);
      rem /= shape[d];
    }
    out[i * W] = (int32_t)rem;
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* implicit-gemm tables (pair_kernels.py:244-261, pairs.py:318-340)          */
/* pair_fwd pre-filled here with -1; pair_bwd may be NULL                    */
/* n_out_eff < n_out implements num_out_act_bound (drops out_row >= bound)   */
/* ------------------------------------------------------------------------ */
int orc_scatter_igemm(const uint8_t* valid, const int32_t* out_row, int64_t kv, int64_t N,
                      int64_t n_out_eff, int32_t* pair_fwd, int32_t* pair_bwd) {
  for (int64_t i = 0; i < kv * n_out_eff; ++i) pair_fwd[i] = -1;
  for (int64_t k = 0; k < kv; ++k) {
    for (int64_t j = 0; j < N; ++j) {
      int64_t off = k * N + j;
      int ok = valid[off] && out_row[off] < n_out_eff;
      if (ok) pair_fwd[k * n_out_eff + out_row[off]] = (int32_t)j;
      if (pair_bwd) pair_bwd[off] = ok ? out_row[off] : -1;
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* mask words + stable sort (pair_kernels.py:169-183, pairs.py:356-392)      */
/* pair_table [kv, n]; pm [n, mic] int32 (wrapped); args [n] int32            */
/* ------------------------------------------------------------------------ */
int orc_mask_split(const int32_t* pair_table, int64_t kv, int64_t n, int64_t mic,
                   int64_t mval, int do_sort, int32_t* pm, int32_t* args) {
  int64_t* words = (int64_t*)calloc((size_t)(n * mic), sizeof(int64_t));
  for (int64_t r = 0; r < n; ++r) {
    for (int64_t k = 0; k < kv; ++k) {
      if (pair_table[k * n + r] >= 0) words[r * mic + k / 32] |= ((int64_t)1) << (k % 32);
    }
    words[r * mic + 0] &= mval;
  }
  int64_t* order = (int64_t*)malloc(sizeof(int64_t) * (size_t)n);
  for (int64_t r = 0; r < n; ++r) order[r] = r;
  if (do_sort) {
    kv_pair* a = (kv_pair*)malloc(sizeof(kv_pair) * (size_t)n);
    kv_pair* t = (kv_pair*)malloc(sizeof(kv_pair) * (size_t)n);
    /* LSD over words: word 0 first, stable, so the highest word is most
       significant (pairs.py:379-384).  For mic == 1 this is one stable sort
       (pairs.py:373-377).  Words are non-negative int64 < 2^32, so signed
       comparison equals unsigned 32-bit order. */
    for (int64_t w = 0; w < mic; ++w) {
      for (int64_t i = 0; i < n; ++i) { a[i].key = words[order[i] * mic + w]; a[i].idx = order[i]; }
      /* stability must follow the current order, so sort positions, not rows */
      for (int64_t i = 0; i < n; ++i) a[i].idx = i;
      merge_sort_pairs(a, t, n);
      int64_t* nord = (int64_t*)malloc(sizeof(int64_t) * (size_t)n);
      for (int64_t i = 0; i < n; ++i) nord[i] = order[a[i].idx];
      memcpy(order, nord, sizeof(int64_t) * (size_t)n);
      free(nord);
    }
    free(a); free(t);
  }
  for (int64_t i = 0; i < n; ++i) {
    args[i] = (int32_t)order[i];
    for (int64_t w = 0; w < mic; ++w) {
      uint32_t v = (uint32_t)(words[order[i] * mic + w] & 0xFFFFFFFFLL);
      pm[i * mic + w] = (int32_t)v; /* two's-complement wrap == pairs.py:388-389 */
    }
  }
  free(order); free(words);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Native [2, kv, N] format (pairs.py:223-239)                               */
/* ------------------------------------------------------------------------ */
int orc_native(const uint8_t* valid, const int32_t* out_row, int64_t kv, int64_t N,
               int32_t* pair, int32_t* counts) {
  for (int64_t i = 0; i < 2 * kv * N; ++i) pair[i] = -1;
  for (int64_t k = 0; k < kv; ++k) {
    int64_t p = 0;
    for (int64_t j = 0; j < N; ++j) {
      if (valid[k * N + j]) {
        pair[k * N + p] = (int32_t)j;
        pair[kv * N + k * N + p] = out_row[k * N + j];
        ++p;
      }
    }
    counts[k] = (int32_t)p;
  }
  return 0;
}

/* Native -> gather tables (pairs.py:429-469); pb may be NULL */
int orc_native_to_tables(const int32_t* pair, int64_t kv, int64_t N, int64_t n_in,
                         int64_t n_out, int inverse, int32_t* pf, int32_t* pb) {
  const int32_t* pin = pair + (inverse ? kv * N : 0);
  const int32_t* pout = pair + (inverse ? 0 : kv * N);
  for (int64_t i = 0; i < kv * n_out; ++i) pf[i] = -1;
  if (pb) for (int64_t i = 0; i < kv * n_in; ++i) pb[i] = -1;
  for (int64_t k = 0; k < kv; ++k) {
    for (int64_t p = 0; p < N; ++p) {
      int32_t a = pin[k * N + p], b = pout[k * N + p];
      if (a >= 0 && b >= 0) {
        pf[k * n_out + b] = a;
        if (pb) pb[k * n_in + a] = b;
      }
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* GEMM contract in fp64 (gemm.py:254-321, :356-426)                         */
/*   out[m,n]  = bias[n] + sum_k sum_c X[pf[k,m],c] * W[n,k,c]               */
/*   dX[j,c]   = sum_k sum_n G[pb[k,j],n] * W[n,k,c]                         */
/*   dW[n,k,c] = sum_{m: pf[k,m]>=0} X[pf[k,m],c] * G[m,n]                   */
/* ------------------------------------------------------------------------ */
int orc_gemm_fwd(const double* X, int64_t C, const double* W, int64_t K, int64_t kv,
                 const int32_t* pf, int64_t n_out, const double* bias, double* out) {
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t m = 0; m < n_out; ++m) {
    double* o = out + m * K;
    for (int64_t n = 0; n < K; ++n) o[n] = bias ? bias[n] : 0.0;
    for (int64_t k = 0; k < kv; ++k) {
      int32_t j = pf[k * n_out + m];
      if (j < 0) continue;
      const double* x = X + (int64_t)j * C;
      for (int64_t n = 0; n < K; ++n) {
        const double* w = W + (n * kv + k) * C;
        double s = 0.0;
        for (int64_t c = 0; c < C; ++c) s += x[c] * w[c];
        o[n] += s;
      }
    }
  }
  return 0;
}

/* fp32 variant of the forward (used only to time the CPU baseline at the
   metric size; the host has no fp16 GEMM) */
int orc_gemm_fwd_f32(const float* X, int64_t C, const float* W, int64_t K, int64_t kv,
                     const int32_t* pf, int64_t n_out, const float* bias, float* out) {
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t m = 0; m < n_out; ++m) {
    float* o = out + m * K;
    for (int64_t n = 0; n < K; ++n) o[n] = bias ? bias[n] : 0.0f;
    for (int64_t k = 0; k < kv; ++k) {
      int32_t j = pf[k * n_out + m];
      if (j < 0) continue;
      const float* x = X + (int64_t)j * C;
      for (int64_t n = 0; n < K; ++n) {
        const float* w = W + (n * kv + k) * C;
        float s = 0.0f;
        for (int64_t c = 0; c < C; ++c) s += x[c] * w[c];
        o[n] += s;
      }
    }
  }
  return 0;
}

int orc_gemm_dgrad(const double* G, int64_t K, const double* W, int64_t kv, int64_t C,
                   const int32_t* pb, int64_t n_in, double* dX) {
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t j = 0; j < n_in; ++j) {
    double* d = dX + j * C;
    for (int64_t c = 0; c < C; ++c) d[c] = 0.0;
    for (int64_t k = 0; k < kv; ++k) {
      int32_t m = pb[k * n_in + j];
      if (m < 0) continue;
      const double* g = G + (int64_t)m * K;
      for (int64_t n = 0; n < K; ++n) {
        const double* w = W + (n * kv + k) * C;
        double gv = g[n];
        for (int64_t c = 0; c < C; ++c) d[c] += gv * w[c];
      }
    }
  }
  return 0;
}

int orc_gemm_wgrad(const double* X, int64_t C, const double* G, int64_t K, int64_t kv,
                   const int32_t* pf, int64_t n_out, double* dW) {
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t k = 0; k < kv; ++k) {
    for (int64_t n = 0; n < K; ++n)
      for (int64_t c = 0; c < C; ++c) dW[(n * kv + k) * C + c] = 0.0;
    for (int64_t m = 0; m < n_out; ++m) {
      int32_t j = pf[k * n_out + m];
      if (j < 0) continue;
      const double* x = X + (int64_t)j * C;
      const double* g = G + m * K;
      for (int64_t n = 0; n < K; ++n) {
        double gv = g[n];
        double* dw = dW + (n * kv + k) * C;
        for (int64_t c = 0; c < C; ++c) dw[c] += x[c] * gv;
      }
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* pooling (pool.py:45-257); FT = accumulator type (float for fp16/fp32     */
/* inputs, double for fp64 inputs), inputs already widened exactly          */
/* ------------------------------------------------------------------------ */
#define DEFINE_POOL(SUF, FT)                                                          \
int orc_maxpool_fwd_##SUF(const FT* X, int64_t C, const int32_t* pf, int64_t kv,     \
                          int64_t n_out, FT* out) {                                  \
  for (int64_t m = 0; m < n_out; ++m)                                                \
    for (int64_t c = 0; c < C; ++c) {                                                \
      FT acc = (FT)0; /* zero init quirk, pool.py:75-76 */                           \
      for (int64_t k = 0; k < kv; ++k) {                                             \
        int32_t j = pf[k * n_out + m];                                               \
        if (j < 0) continue;                                                         \
        FT v = X[(int64_t)j * C + c];                                                \
        acc = v > acc ? v : acc;                                                     \
      }                                                                              \
      out[m * C + c] = acc;                                                          \
    }                                                                                \
  return 0;                                                                          \
}                                                                                    \
int orc_maxpool_bwd_##SUF(const FT* X, const FT* OUT, const FT* G, int64_t C,        \
                          const int32_t* pb, int64_t kv, int64_t n_in, FT* dX) {     \
  for (int64_t j = 0; j < n_in; ++j)                                                 \
    for (int64_t c = 0; c < C; ++c) {                                                \
      FT acc = (FT)0;                                                                \
      FT f = X[j * C + c];                                                           \
      for (int64_t k = 0; k < kv; ++k) {                                             \
        int32_t m = pb[k * n_in + j];                                                \
        if (m < 0) continue;                                                         \
        if (OUT[(int64_t)m * C + c] == f) acc += G[(int64_t)m * C + c];              \
      }                                                                              \
      dX[j * C + c] = acc;                                                           \
    }                                                                                \
  return 0;                                                                          \
}                                                                                    \
int orc_avgpool_fwd_##SUF(const FT* X, int64_t C, const int32_t* pf, int64_t kv,     \
                          int64_t n_out, FT* out, int32_t* count) {                  \
  for (int64_t m = 0; m < n_out; ++m) {                                              \
    int32_t cnt = 0;                                                                 \
    for (int64_t k = 0; k < kv; ++k) cnt += pf[k * n_out + m] >= 0;                  \
    for (int64_t c = 0; c < C; ++c) {                                                \
      FT acc = (FT)0;                                                                \
      for (int64_t k = 0; k < kv; ++k) {                                             \
        int32_t j = pf[k * n_out + m];                                               \
        if (j >= 0) acc += X[(int64_t)j * C + c];                                    \
      }                                                                              \
      out[m * C + c] = acc / (FT)(cnt > 1 ? cnt : 1);                                \
    }                                                                                \
    count[m] = cnt;                                                                  \
  }                                                                                  \
  return 0;                                                                          \
}                                                                                    \
int orc_avgpool_bwd_##SUF(const FT* G, const int32_t* count, int64_t C,              \
                          const int32_t* pb, int64_t kv, int64_t n_in, FT* dX) {     \
  for (int64_t j = 0; j < n_in; ++j)                                                 \
    for (int64_t c = 0; c < C; ++c) {                                                \
      FT acc = (FT)0;                                                                \
      for (int64_t k = 0; k < kv; ++k) {                                             \
        int32_t m = pb[k * n_in + j];                                                \
        if (m < 0) continue;                                                         \
        /* multiplies by the window count: upstream quirk, pool.py:251-252 */        \
        acc += G[(int64_t)m * C + c] * (FT)count[m];                                 \
      }                                                                              \
      dX[j * C + c] = acc;                                                           \
    }                                                                                \
  return 0;                                                                          \
}

DEFINE_POOL(f32, float)
DEFINE_POOL(f64, double)

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void orc_set_num_threads(int n) {
#ifdef _OPENMP
  omp_set_num_threads(n);
#else
  (void)n;
#endif
}
