// CPU kernels of the philtorch operators (the torch.library CPU key):
// h[t] = A[t] h[t-1] + x[t], h[-1] = zi, for a state of any order M, and
// the fused adjoint of the same recurrence.
//
// These replace the reference's CPU extension (philtorch/csrc/
// host_recurN.cpp:81-140,236-281, host_lti_recur.cpp:4-80,
// host_lti_recurN.cpp:4-108) and, for the backward ops, its composite
// closures (philtorch/__init__.py:34-148).  Rows run in parallel; each row
// runs serially in time with the reference's arithmetic: per step and state
// component, the products A[i][j] h[j] summed from zero in j order, then
// added to x[i] (so a scalar step is x + a h_prev).  The forward results are
// therefore the reference CPU results bit for bit, in every dtype the
// reference dispatches, half and bfloat16 included (no fused multiply-add:
// this file is built for the baseline x86-64 target).  The backward runs the
// adjoint lambda[t] = g[t] + A[t+1]^H lambda[t+1] directly, in one pass per
// row, instead of the reference's flipped, rolled and conjugated copies.
//
// No device code and no torch types in the kernels: element types are
// float, double, c10::complex<float>, c10::complex<double>, int64_t and the
// 16-bit c10::Half and c10::BFloat16, whose operators round to the type after
// every multiply and add, as the reference's loops in those dtypes do; the
// caller passes contiguous buffers and a `parallel_rows(n, fn)` runner.
#pragma once

#include <c10/util/BFloat16.h>
#include <c10/util/Half.h>
#include <c10/util/complex.h>

#include <cstdint>
#include <cstring>
#include <vector>

namespace phs_cpu {

template <typename T>
inline T conj_of(T v) {
  return v;
}

// Accumulator of the backward's sums over steps or rows (coefficient
// gradients of shared or time-invariant coefficients, grad_zi): float for
// the 16-bit types, as the reference's closures form those sums with
// matmul / vecdot, which accumulate 16-bit operands in float; the element
// type otherwise.
template <typename S>
struct AccOf {
  using type = S;
};
template <>
struct AccOf<c10::Half> {
  using type = float;
};
template <>
struct AccOf<c10::BFloat16> {
  using type = float;
};
template <typename S>
inline typename AccOf<S>::type acc_of(S v) {
  return typename AccOf<S>::type(v);
}
template <typename R>
inline c10::complex<R> conj_of(c10::complex<R> v) {
  return c10::complex<R>(v.real(), -v.imag());
}

// Operand layout of A: element (row b, step t, i, j) at
// A[b * a_row + t * a_step + i * M + j]; a_row == 0 shares A across rows,
// a_step == 0 holds A constant in time (LTI).  `direct`: a scalar step is
// x + a h (the reference's lti_recur loop) rather than x + (0 + a h) (its
// generic M x M loop at M = 1); the two differ only in the sign of a zero.
struct Layout {
  int64_t B, T, M;
  int64_t a_row, a_step;
  bool direct = false;
};

// Forward scan of row b.
template <typename S>
inline void scan_row(const Layout &L, int64_t b, const S *A, const S *zi, const S *x, S *y) {
  const int64_t M = L.M, T = L.T;
  const S *Ab = A + b * L.a_row;
  const S *xb = x + b * T * M;
  S *yb = y + b * T * M;
  if (M == 1 && L.direct) {
    S h = zi[b];
    for (int64_t t = 0; t < T; ++t) {
      h = xb[t] + Ab[t * L.a_step] * h;
      yb[t] = h;
    }
    return;
  }
  const S *hp = zi + b * M;
  for (int64_t t = 0; t < T; ++t) {
    const S *At = Ab + t * L.a_step;
    S *hc = yb + t * M;
    for (int64_t i = 0; i < M; ++i) {
      S sum = S(0);
      for (int64_t j = 0; j < M; ++j) sum += At[i * M + j] * hp[j];
      hc[i] = xb[t * M + i] + sum;
    }
    hp = hc;
  }
}

template <typename S, class Par>
void scan_fwd(const Layout &L, const S *A, const S *zi, const S *x, S *y, Par &&parallel_rows) {
  parallel_rows(L.B, [&](int64_t b) { scan_row(L, b, A, zi, x, y); });
}

// Adjoint of row b: lambda (written to gx, the gradient w.r.t. x), grad_zi
// and, per step, the coefficient gradient lambda[t] conj(h[t-1])^T, which
// `on_step(t, lam, hprev)` receives.  lambda[t] = g[t] + A[t+1]^H lambda[t+1]
// with lambda[T-1] = g[T-1]; grad_zi = A[0]^H lambda[0].
template <typename S, class OnStep>
inline void adjoint_row(const Layout &L, int64_t b, const S *A, const S *zi, const S *y, const S *g, S *gx,
                        S *gzi, OnStep &&on_step) {
  const int64_t M = L.M, T = L.T;
  const S *Ab = A + b * L.a_row;
  const S *gb = g + b * T * M;
  const S *yb = y + b * T * M;
  S *lb = gx + b * T * M;
  for (int64_t t = T - 1; t >= 0; --t) {
    S *lam = lb + t * M;
    if (t == T - 1) {
      for (int64_t i = 0; i < M; ++i) lam[i] = gb[t * M + i];
    } else {
      const S *An = Ab + (t + 1) * L.a_step;
      const S *ln = lam + M;
      for (int64_t i = 0; i < M; ++i) {
        S sum = S(0);
        for (int64_t j = 0; j < M; ++j) sum += conj_of(An[j * M + i]) * ln[j];
        lam[i] = gb[t * M + i] + sum;
      }
    }
    on_step(t, lam, t == 0 ? zi + b * M : yb + (t - 1) * M);
  }
  if (gzi && T > 0) {
    using Acc = typename AccOf<S>::type;
    for (int64_t i = 0; i < M; ++i) {
      Acc sum = Acc(0);
      for (int64_t j = 0; j < M; ++j) sum += acc_of(conj_of(Ab[j * M + i])) * acc_of(lb[j]);
      gzi[b * M + i] = S(sum);
    }
  }
}

// Backward of scan_fwd.  gA holds, by the layout of A:
//   a_step != 0, a_row != 0: per row and step [B, T, M, M]
//   a_step != 0, a_row == 0: per step, summed over rows in row order [T, M, M]
//   a_step == 0, a_row != 0: per row, summed over steps [B, M, M]
//   a_step == 0, a_row == 0: one matrix, summed over rows and steps [M, M]
// gx (the adjoint lambda) is always written; gA and gzi may be null.
template <typename S, class Par>
void scan_bwd(const Layout &L, const S *A, const S *zi, const S *y, const S *g, S *gx, S *gA, S *gzi,
              Par &&parallel_rows) {
  using Acc = typename AccOf<S>::type;
  const int64_t B = L.B, T = L.T, M = L.M, MM = M * M;
  const bool tv = L.a_step != 0, shared = L.a_row == 0;
  if (gA && tv && !shared) {
    parallel_rows(B, [&](int64_t b) {
      S *gAb = gA + b * T * MM;
      adjoint_row(L, b, A, zi, y, g, gx, gzi, [&](int64_t t, const S *lam, const S *hp) {
        for (int64_t i = 0; i < M; ++i)
          for (int64_t j = 0; j < M; ++j) gAb[t * MM + i * M + j] = lam[i] * conj_of(hp[j]);
      });
    });
    return;
  }
  if (gA && !tv) {
    // per-row sums over time, then (shared A) over rows in row order
    std::vector<Acc> rows(size_t(B * MM));
    parallel_rows(B, [&](int64_t b) {
      Acc *dst = rows.data() + b * MM;
      for (int64_t k = 0; k < MM; ++k) dst[k] = Acc(0);
      adjoint_row(L, b, A, zi, y, g, gx, gzi, [&](int64_t, const S *lam, const S *hp) {
        for (int64_t i = 0; i < M; ++i)
          for (int64_t j = 0; j < M; ++j) dst[i * M + j] += acc_of(lam[i]) * acc_of(conj_of(hp[j]));
      });
      if (!shared)
        for (int64_t k = 0; k < MM; ++k) gA[b * MM + k] = S(dst[k]);
    });
    if (shared) {
      for (int64_t k = 0; k < MM; ++k) {
        Acc sum = Acc(0);
        for (int64_t b = 0; b < B; ++b) sum += rows[b * MM + k];
        gA[k] = S(sum);
      }
    }
    return;
  }
  // lambda for every row first; a coefficient shared across rows then sums
  // the rows' products per step, in row order, over steps in parallel
  parallel_rows(B, [&](int64_t b) { adjoint_row(L, b, A, zi, y, g, gx, gzi, [](int64_t, const S *, const S *) {}); });
  if (!gA) return;
  parallel_rows(T, [&](int64_t t) {
    thread_local std::vector<Acc> dst;
    dst.assign(size_t(MM), Acc(0));
    for (int64_t b = 0; b < B; ++b) {
      const S *lam = gx + (b * T + t) * M;
      const S *hp = t == 0 ? zi + b * M : y + (b * T + t - 1) * M;
      for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < M; ++j) dst[i * M + j] += acc_of(lam[i]) * acc_of(conj_of(hp[j]));
    }
    for (int64_t k = 0; k < MM; ++k) gA[t * MM + k] = S(dst[k]);
  });
}

}  // namespace phs_cpu
