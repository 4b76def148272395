/*
 * CPU oracle for the linear-recurrence core — TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C with OpenMP over the batch, the algorithm of
 * philtorch's CPU extension and of the composite backward closures that
 * philtorch registers with torch.library.  It is the checker the GPU path is
 * compared against and the timed CPU baseline ("port") of bench.py.  Nothing
 * in the product (philtorch_amd/) links, loads or calls it.
 *
 * Forward ops, all `h[t] = A[t] h[t-1] + x[t]`, `h[-1] = zi`, output = states
 * after consuming x[t]:
 *   recurN      philtorch/csrc/host_recurN.cpp:236-281 (mat_recur_N_order_cpu_omp_impl)
 *               -> host_batch_mat_recur_N_order_omp :81-111 / host_share_... :113-140.
 *               The reference pads A with one leading zero step (:254), prepends zi
 *               to x (:255), runs t = 1..T serially per batch row, and slices the
 *               first step off (:279).  M = 1 is the LPV scalar scan; M = 2 is recur2.
 *   lti_recur   philtorch/csrc/host_lti_recur.cpp:42-80 (batched a[b] :4-22,
 *               shared scalar a :24-40).
 *   lti_recurN  philtorch/csrc/host_lti_recurN.cpp:63-108 (batched :5-33,
 *               shared :36-61).  M = 2 is lti_recur2.
 *
 * Backward closures (reverse-time scan of the same form):
 *   recurN      philtorch/__init__.py:34-73  (_recurN_backward)
 *   lti_recurN  philtorch/__init__.py:76-112 (_lti_recurN_backward)
 *   lti_recur   philtorch/__init__.py:115-148 (_lti_recur_backward)
 * Each is restated step by step: conj-transpose of A, roll(-1) along time,
 * flip, a forward scan with zero initial state, then grad_zi, grad_x and the
 * outer-product / reduced grad_A.
 *
 * Pinning (tests/test_oracle.py): closed forms (a=0, a=1, x=0, constant a vs
 * scipy.signal.lfilter), an independent explicit-product formula, the README
 * Fibonacci known answer through lti_recur2 in int64, biquads vs
 * scipy.signal.lfilter, finite differences and the adjoint identity for the
 * backward, golden vectors written by the reference's own CPU extension
 * (tests/golden/), and oracle/_ref where that builds.
 */
#include <complex.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef float _Complex c64_t;
typedef double _Complex c128_t;
typedef long long i64_t;

static inline float conj_f32(float v) { return v; }
static inline double conj_f64(double v) { return v; }
static inline c64_t conj_c64(c64_t v) { return conjf(v); }
static inline c128_t conj_c128(c128_t v) { return conj(v); }
static inline i64_t conj_i64(i64_t v) { return v; }

static void set_threads(int nthreads) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
}

#define DEFINE_ORACLE(SFX, S)                                                     \
  /* host_recurN.cpp:81-140 — serial t per batch row, OMP over rows. */          \
  static void mat_recur_loop_##SFX(int64_t B, int64_t T1, int64_t M,              \
                                   const S *Apad, int A_batched, S *H) {          \
    int64_t b;                                                                    \
    _Pragma("omp parallel for") for (b = 0; b < B; ++b) {                         \
      const S *A_b = A_batched ? Apad + b * T1 * M * M : Apad;                    \
      S *H_b = H + b * T1 * M;                                                    \
      for (int64_t t = 1; t < T1; ++t) {                                          \
        const S *A_bt = A_b + t * M * M;                                          \
        const S *Hp = H_b + (t - 1) * M;                                          \
        S *Hc = H_b + t * M;                                                      \
        for (int64_t i = 0; i < M; ++i) {                                         \
          S sum = 0;                                                              \
          const S *Arow = A_bt + i * M;                                           \
          for (int64_t j = 0; j < M; ++j) sum += Arow[j] * Hp[j];                 \
          Hc[i] += sum;                                                           \
        }                                                                         \
      }                                                                           \
    }                                                                             \
  }                                                                               \
                                                                                  \
  /* host_recurN.cpp:236-281: pad A (:254), cat(zi, x) (:255), loop, slice. */    \
  int oracle_recurN_##SFX(int64_t B, int64_t T, int64_t M, const S *A,            \
                          int A_batched, const S *zi, const S *x, S *y,           \
                          int nthreads) {                                         \
    set_threads(nthreads);                                                        \
    int64_t T1 = T + 1, MM = M * M, nA = A_batched ? B : 1;                       \
    S *Apad = (S *)malloc(sizeof(S) * nA * T1 * MM);                              \
    S *H = (S *)malloc(sizeof(S) * B * T1 * M);                                   \
    if (!Apad || !H) { free(Apad); free(H); return 1; }                           \
    for (int64_t b = 0; b < nA; ++b) {                                            \
      memset(Apad + b * T1 * MM, 0, sizeof(S) * MM);                              \
      memcpy(Apad + b * T1 * MM + MM, A + b * T * MM, sizeof(S) * T * MM);        \
    }                                                                             \
    for (int64_t b = 0; b < B; ++b) {                                             \
      memcpy(H + b * T1 * M, zi + b * M, sizeof(S) * M);                          \
      memcpy(H + b * T1 * M + M, x + b * T * M, sizeof(S) * T * M);               \
    }                                                                             \
    mat_recur_loop_##SFX(B, T1, M, Apad, A_batched, H);                           \
    for (int64_t b = 0; b < B; ++b)                                               \
      memcpy(y + b * T * M, H + b * T1 * M + M, sizeof(S) * T * M);               \
    free(Apad);                                                                   \
    free(H);                                                                      \
    return 0;                                                                     \
  }                                                                               \
                                                                                  \
  /* host_lti_recurN.cpp:5-61 (A [M,M] shared or [B,M,M]). */                     \
  int oracle_lti_recurN_##SFX(int64_t B, int64_t T, int64_t M, const S *A,        \
                              int A_batched, const S *zi, const S *x, S *y,       \
                              int nthreads) {                                     \
    set_threads(nthreads);                                                        \
    int64_t T1 = T + 1, MM = M * M;                                               \
    S *H = (S *)malloc(sizeof(S) * B * T1 * M);                                   \
    if (!H) return 1;                                                             \
    for (int64_t b = 0; b < B; ++b) {                                             \
      memcpy(H + b * T1 * M, zi + b * M, sizeof(S) * M);                          \
      memcpy(H + b * T1 * M + M, x + b * T * M, sizeof(S) * T * M);               \
    }                                                                             \
    int64_t b;                                                                    \
    _Pragma("omp parallel for") for (b = 0; b < B; ++b) {                         \
      const S *A_b = A_batched ? A + b * MM : A;                                  \
      S *H_b = H + b * T1 * M;                                                    \
      for (int64_t t = 1; t < T1; ++t) {                                          \
        const S *Hp = H_b + (t - 1) * M;                                          \
        S *Hc = H_b + t * M;                                                      \
        for (int64_t i = 0; i < M; ++i) {                                         \
          S sum = 0;                                                              \
          const S *Arow = A_b + i * M;                                            \
          for (int64_t j = 0; j < M; ++j) sum += Arow[j] * Hp[j];                 \
          Hc[i] += sum;                                                           \
        }                                                                         \
      }                                                                           \
    }                                                                             \
    for (int64_t bb = 0; bb < B; ++bb)                                            \
      memcpy(y + bb * T * M, H + bb * T1 * M + M, sizeof(S) * T * M);             \
    free(H);                                                                      \
    return 0;                                                                     \
  }                                                                               \
                                                                                  \
  /* host_lti_recur.cpp:42-80: a_numel == B -> per-row a[b], else a[0]. */        \
  int oracle_lti_recur_##SFX(int64_t B, int64_t T, const S *a, int64_t a_numel,   \
                             const S *zi, const S *x, S *y, int nthreads) {       \
    set_threads(nthreads);                                                        \
    int64_t T1 = T + 1;                                                           \
    S *H = (S *)malloc(sizeof(S) * B * T1);                                       \
    if (!H) return 1;                                                             \
    for (int64_t b = 0; b < B; ++b) {                                             \
      H[b * T1] = zi[b];                                                          \
      memcpy(H + b * T1 + 1, x + b * T, sizeof(S) * T);                           \
    }                                                                             \
    int batched = (a_numel == B);                                                 \
    int64_t b;                                                                    \
    _Pragma("omp parallel for") for (b = 0; b < B; ++b) {                         \
      const S a_b = batched ? a[b] : a[0];                                        \
      S *out_b = H + b * T1;                                                      \
      for (int64_t t = 1; t < T1; ++t) out_b[t] += a_b * out_b[t - 1];            \
    }                                                                             \
    for (int64_t bb = 0; bb < B; ++bb)                                            \
      memcpy(y + bb * T, H + bb * T1 + 1, sizeof(S) * T);                         \
    free(H);                                                                      \
    return 0;                                                                     \
  }                                                                               \
                                                                                  \
  /* philtorch/__init__.py:34-73 (_recurN_backward).  Any of gA/gzi/gx may be     \
     NULL (needs_input_grad false).  gA is [B,T,M,M] when A is batched, else      \
     [T,M,M] reduced over the batch. */                                           \
  int oracle_recurN_bwd_##SFX(int64_t B, int64_t T, int64_t M, const S *A,        \
                              int A_batched, const S *zi, const S *y,             \
                              const S *gy, S *gA, S *gzi, S *gx, int nthreads) {  \
    set_threads(nthreads);                                                        \
    int64_t MM = M * M, nA = A_batched ? B : 1;                                   \
    /* AmT = A.mT.conj_physical() (:41) */                                        \
    S *AmT = (S *)malloc(sizeof(S) * nA * T * MM);                                \
    /* roll(AmT, -1, time) (:42) then flip(time) (:47) */                         \
    S *Arf = (S *)malloc(sizeof(S) * nA * T * MM);                                \
    S *gflip = (S *)malloc(sizeof(S) * B * T * M);                                \
    S *z0 = (S *)calloc((size_t)(B * M), sizeof(S));                              \
    S *lam_f = (S *)malloc(sizeof(S) * B * T * M);                                \
    if (!AmT || !Arf || !gflip || !z0 || !lam_f) return 1;                        \
    for (int64_t n = 0; n < nA * T; ++n)                                          \
      for (int64_t i = 0; i < M; ++i)                                             \
        for (int64_t j = 0; j < M; ++j)                                           \
          AmT[n * MM + i * M + j] = conj_##SFX(A[n * MM + j * M + i]);            \
    for (int64_t b = 0; b < nA; ++b)                                              \
      for (int64_t s = 0; s < T; ++s) {                                           \
        int64_t t_roll = T - 1 - s;            /* flip */                         \
        int64_t t_src = (t_roll + 1) % T;      /* roll(-1) wraps */               \
        memcpy(Arf + (b * T + s) * MM, AmT + (b * T + t_src) * MM,                \
               sizeof(S) * MM);                                                   \
      }                                                                           \
    for (int64_t b = 0; b < B; ++b)                                               \
      for (int64_t s = 0; s < T; ++s)                                             \
        memcpy(gflip + (b * T + s) * M, gy + (b * T + T - 1 - s) * M,             \
               sizeof(S) * M);                                                    \
    /* flipped_grad_x = recur(Arf, zeros_like(zi), grad_y.flip(1)) (:46-50) */    \
    int rc = oracle_recurN_##SFX(B, T, M, Arf, A_batched, z0, gflip, lam_f,       \
                                 nthreads);                                       \
    if (rc) return rc;                                                            \
    /* grad_zi = AmT[...,0,:,:] @ flipped_grad_x[:, -1] (:53) */                  \
    if (gzi)                                                                      \
      for (int64_t b = 0; b < B; ++b) {                                           \
        const S *A0 = AmT + (A_batched ? b * T * MM : 0);                         \
        const S *l0 = lam_f + (b * T + T - 1) * M;                                \
        for (int64_t i = 0; i < M; ++i) {                                         \
          S s = 0;                                                                \
          for (int64_t j = 0; j < M; ++j) s += A0[i * M + j] * l0[j];             \
          gzi[b * M + i] = s;                                                     \
        }                                                                         \
      }                                                                           \
    /* grad_x = flipped_grad_x.flip(1) (:56) */                                   \
    if (gx)                                                                       \
      for (int64_t b = 0; b < B; ++b)                                             \
        for (int64_t t = 0; t < T; ++t)                                           \
          memcpy(gx + (b * T + t) * M, lam_f + (b * T + T - 1 - t) * M,           \
                 sizeof(S) * M);                                                  \
    /* grad_A: padded_y = cat(zi, y[:, :-1]) (:59-60); outer products (:62-69) */ \
    if (gA) {                                                                     \
      if (!A_batched) memset(gA, 0, sizeof(S) * T * MM);                          \
      for (int64_t b = 0; b < B; ++b)                                             \
        for (int64_t t = 0; t < T; ++t) {                                         \
          const S *yp = t == 0 ? zi + b * M : y + (b * T + t - 1) * M;            \
          const S *lt = lam_f + (b * T + T - 1 - t) * M;                          \
          S *dst = A_batched ? gA + (b * T + t) * MM : gA + t * MM;               \
          for (int64_t i = 0; i < M; ++i)                                         \
            for (int64_t j = 0; j < M; ++j) {                                     \
              if (A_batched)                                                      \
                dst[i * M + j] = lt[i] * conj_##SFX(yp[j]);                       \
              else                                                                \
                dst[i * M + j] += lt[i] * conj_##SFX(yp[j]);                      \
            }                                                                     \
        }                                                                         \
    }                                                                             \
    free(AmT); free(Arf); free(gflip); free(z0); free(lam_f);                     \
    return 0;                                                                     \
  }                                                                               \
                                                                                  \
  /* philtorch/__init__.py:76-112 (_lti_recurN_backward).  gA is [B,M,M] when A   \
     is batched, [M,M] when shared (summed over batch and time). */               \
  int oracle_lti_recurN_bwd_##SFX(int64_t B, int64_t T, int64_t M, const S *A,    \
                                  int A_batched, const S *zi, const S *y,         \
                                  const S *gy, S *gA, S *gzi, S *gx,              \
                                  int nthreads) {                                 \
    set_threads(nthreads);                                                        \
    int64_t MM = M * M, nA = A_batched ? B : 1;                                   \
    S *AmT = (S *)malloc(sizeof(S) * nA * MM);                                    \
    S *gflip = (S *)malloc(sizeof(S) * B * T * M);                                \
    S *z0 = (S *)calloc((size_t)(B * M), sizeof(S));                              \
    S *lam_f = (S *)malloc(sizeof(S) * B * T * M);                                \
    if (!AmT || !gflip || !z0 || !lam_f) return 1;                                \
    for (int64_t n = 0; n < nA; ++n)                                              \
      for (int64_t i = 0; i < M; ++i)                                             \
        for (int64_t j = 0; j < M; ++j)                                           \
          AmT[n * MM + i * M + j] = conj_##SFX(A[n * MM + j * M + i]);            \
    for (int64_t b = 0; b < B; ++b)                                               \
      for (int64_t s = 0; s < T; ++s)                                             \
        memcpy(gflip + (b * T + s) * M, gy + (b * T + T - 1 - s) * M,             \
               sizeof(S) * M);                                                    \
    /* flipped_grad_x = runner(AmT, zeros_like(zi), grad_y.flip(1)) (:92) */      \
    int rc = oracle_lti_recurN_##SFX(B, T, M, AmT, A_batched, z0, gflip, lam_f,   \
                                     nthreads);                                   \
    if (rc) return rc;                                                            \
    if (gzi) /* (:95) */                                                          \
      for (int64_t b = 0; b < B; ++b) {                                           \
        const S *A0 = AmT + (A_batched ? b * MM : 0);                             \
        const S *l0 = lam_f + (b * T + T - 1) * M;                                \
        for (int64_t i = 0; i < M; ++i) {                                         \
          S s = 0;                                                                \
          for (int64_t j = 0; j < M; ++j) s += A0[i * M + j] * l0[j];             \
          gzi[b * M + i] = s;                                                     \
        }                                                                         \
      }                                                                           \
    if (gx) /* (:98) */                                                           \
      for (int64_t b = 0; b < B; ++b)                                             \
        for (int64_t t = 0; t < T; ++t)                                           \
          memcpy(gx + (b * T + t) * M, lam_f + (b * T + T - 1 - t) * M,           \
                 sizeof(S) * M);                                                  \
    if (gA) { /* (:100-108): sum_t lambda_t conj(y_{t-1})^T */                    \
      memset(gA, 0, sizeof(S) * nA * MM);                                         \
      for (int64_t b = 0; b < B; ++b) {                                           \
        S *dst = gA + (A_batched ? b * MM : 0);                                   \
        for (int64_t t = 0; t < T; ++t) {                                         \
          const S *yp = t == 0 ? zi + b * M : y + (b * T + t - 1) * M;            \
          const S *lt = lam_f + (b * T + T - 1 - t) * M;                          \
          for (int64_t i = 0; i < M; ++i)                                         \
            for (int64_t j = 0; j < M; ++j)                                       \
              dst[i * M + j] += lt[i] * conj_##SFX(yp[j]);                        \
        }                                                                         \
      }                                                                           \
    }                                                                             \
    free(AmT); free(gflip); free(z0); free(lam_f);                                \
    return 0;                                                                     \
  }                                                                               \
                                                                                  \
  /* philtorch/__init__.py:115-148 (_lti_recur_backward).  ga has a_numel        \
     entries: per-row vecdot when a is [B], full sum when a is a scalar. */       \
  int oracle_lti_recur_bwd_##SFX(int64_t B, int64_t T, const S *a,                \
                                 int64_t a_numel, const S *zi, const S *y,        \
                                 const S *gy, S *ga, S *gzi, S *gx,               \
                                 int nthreads) {                                  \
    set_threads(nthreads);                                                        \
    int batched = (a_numel == B);                                                 \
    int64_t na = batched ? B : 1;                                                 \
    S *ac = (S *)malloc(sizeof(S) * na);                                          \
    S *bp = (S *)malloc(sizeof(S) * B);                                           \
    S *gin = (S *)malloc(sizeof(S) * B * (T > 1 ? T - 1 : 1));                    \
    S *lam_f = (S *)malloc(sizeof(S) * B * T); /* flipped lambda */               \
    S *tmp = (S *)malloc(sizeof(S) * B * (T > 1 ? T - 1 : 1));                    \
    if (!ac || !bp || !gin || !lam_f || !tmp) return 1;                           \
    for (int64_t n = 0; n < na; ++n) ac[n] = conj_##SFX(a[n]);                    \
    /* bp_init = grad_out[:, -1] (:121) */                                        \
    for (int64_t b = 0; b < B; ++b) bp[b] = gy[b * T + T - 1];                    \
    /* lti_recur(conj(a), bp_init, grad_out[:, :-1].flip(1)) (:125-129) */        \
    for (int64_t b = 0; b < B; ++b)                                               \
      for (int64_t s = 0; s < T - 1; ++s)                                         \
        gin[b * (T - 1) + s] = gy[b * T + T - 2 - s];                             \
    if (T > 1) {                                                                  \
      int rc = oracle_lti_recur_##SFX(B, T - 1, ac, na, bp, gin, tmp, nthreads);  \
      if (rc) return rc;                                                          \
    }                                                                             \
    /* flipped_grad_x = cat(bp_init, scan) (:122-132) */                          \
    for (int64_t b = 0; b < B; ++b) {                                             \
      lam_f[b * T] = bp[b];                                                       \
      for (int64_t s = 0; s < T - 1; ++s)                                         \
        lam_f[b * T + 1 + s] = tmp[b * (T - 1) + s];                              \
    }                                                                             \
    if (gzi) /* flipped_grad_x[:, -1] * conj(a) (:135) */                         \
      for (int64_t b = 0; b < B; ++b)                                             \
        gzi[b] = lam_f[b * T + T - 1] * ac[batched ? b : 0];                      \
    if (gx) /* (:138) */                                                          \
      for (int64_t b = 0; b < B; ++b)                                             \
        for (int64_t t = 0; t < T; ++t) gx[b * T + t] = lam_f[b * T + T - 1 - t]; \
    if (ga) { /* vecdot(padded_out, lambda) = sum conj(padded_out) * lambda */    \
      for (int64_t n = 0; n < na; ++n) ga[n] = 0;                                 \
      for (int64_t b = 0; b < B; ++b) {                                           \
        S acc = 0;                                                                \
        for (int64_t t = 0; t < T; ++t) {                                         \
          S yp = t == 0 ? zi[b] : y[b * T + t - 1];                               \
          acc += conj_##SFX(yp) * lam_f[b * T + T - 1 - t];                       \
        }                                                                         \
        ga[batched ? b : 0] += acc;                                               \
      }                                                                           \
    }                                                                             \
    free(ac); free(bp); free(gin); free(lam_f); free(tmp);                        \
    return 0;                                                                     \
  }

DEFINE_ORACLE(f32, float)
DEFINE_ORACLE(f64, double)
DEFINE_ORACLE(c64, c64_t)
DEFINE_ORACLE(c128, c128_t)
DEFINE_ORACLE(i64, i64_t)
