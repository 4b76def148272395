// Zero-phase filtering of one second-order section per row: the edge work
// around the two cascade passes (philtorch/lti/filtering.py:413-484 filtfilt,
// with lfilter_zi :107-142, for a biquad).
//
// The reference pads x by e samples at both ends (F.pad, `padmode`), runs
// lfilter over the padded row from the steady state zi * ext[0]
// (zi = (I - A)^-1 c), runs lfilter again over the reversed output from
// zi * y1[last], and trims and flips.  Here:
//
//  * pass 1 is the forward cascade kernel over x itself; its entry state is
//    the steady state advanced over the front pad (filtfilt_pre_kernel);
//  * the back pad, whose outputs only feed pass 2, is stepped from pass 1's
//    final state (filtfilt_mid_kernel);
//  * pass 2 is the adjoint cascade kernel (time reversed, transposed section:
//    m <- A^T m + e0 v, out = c.m + b0 v).  Its transfer function is the
//    section's own, b0 + e0^T (zI - A)^-1 c = b0 + c^T (zI - A^T)^-1 e0, so it
//    filters the reversed row exactly as lfilter does; its steady state for a
//    constant input y0 is m* = (I - A^T)^-1 e0 y0 = y0 / (1 + a1 + a2) (1, 1),
//    and both steady states give the same future outputs, because
//    e0^T A^j (I - A)^-1 c = c^T (A^T)^j (I - A^T)^-1 e0 for every j.  The
//    reversed pass over the back pad folds into its entry state
//        m_e = (A^T)^e m*(y1b[e-1]) + sum_j (A^T)^j e0 y1b[j],
//    and its outputs are written in place of the flip and the trim.
//
// A section with a pole at z = 1 (1 + a1 + a2 = 0) has no steady state: the
// reference's linalg.solve raises, here the output is not finite.
#pragma once

#include "phs_sos.hpp"

namespace phs {

// padmode codes (PHS_PAD_* in philscan.h): torch.nn.functional.pad modes
constexpr int kPadConstant = 0;   // zeros
constexpr int kPadReplicate = 1;  // edge value
constexpr int kPadReflect = 2;    // mirror without repeating the edge
constexpr int kPadCircular = 3;   // wrap around

template <typename E>
struct FiltfiltEdge {
  const E *b, *a;          // numerator [rows, nb], denominator after its leading 1 [rows, na]
  int nb, na;              // 1..3, 1..2
  E *sos;                  // [rows, 6] section rows (b0 b1 b2 1 a1 a2): written by the pre kernel
  int64_t rows;            // 1 (coefficients shared by every row) or B
  const E *x;              // [B, T]
  const E *y1;             // [B, T] pass 1 output (mid kernel, e = 0 only)
  const E *zf1;            // [B, 2] pass 1 final state (mid kernel)
  E *state;                // [B, 2] out: pass 1 entry state (pre) / pass 2 entry state (mid)
  int64_t B, T, e;
  int mode;
};

// ext[j] for j in [0, e): the front pad (e < T)
template <typename E>
__device__ __forceinline__ E pad_front(const E *x, int64_t T, int64_t e, int mode, int64_t j) {
  switch (mode) {
    case kPadReplicate: return x[0];
    case kPadReflect: return x[e - j];
    case kPadCircular: return x[T - e + j];
    default: return E(0);
  }
}

// ext[T + e + j] for j in [0, e): the back pad (e < T)
template <typename E>
__device__ __forceinline__ E pad_back(const E *x, int64_t T, int mode, int64_t j) {
  switch (mode) {
    case kPadReplicate: return x[T - 1];
    case kPadReflect: return x[T - 2 - j];
    case kPadCircular: return x[j];
    default: return E(0);
  }
}

// The section of row b: b and a zero-padded to second order (a first-order
// filter is the biquad with b2 = a2 = 0, whose second state stays zero).
template <typename E>
__device__ __forceinline__ void section_row(const FiltfiltEdge<E> &a, int64_t r, E (&row)[6]) {
  const E *bp = a.b + r * a.nb, *ap = a.a + r * a.na;
  row[0] = bp[0];
  row[1] = a.nb > 1 ? bp[1] : E(0);
  row[2] = a.nb > 2 ? bp[2] : E(0);
  row[3] = E(1);
  row[4] = ap[0];
  row[5] = a.na > 1 ? ap[1] : E(0);
}

template <typename E>
__device__ __forceinline__ SosSec<E> edge_section(const FiltfiltEdge<E> &a, int64_t b) {
  E row[6];
  section_row(a, a.rows == 1 ? 0 : b, row);
  return load_sec(row, 0);
}

// Pass 1 entry state: zi * ext[0], stepped over the e front-pad samples; the
// section rows both cascade passes read.
template <typename E>
__global__ void filtfilt_pre_kernel(FiltfiltEdge<E> a) {
  using C = typename Wide<E>::type;
  const int64_t b = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= a.B) return;
  if (b < a.rows) {
    E row[6];
    section_row(a, b, row);
#pragma unroll
    for (int i = 0; i < 6; ++i) a.sos[b * 6 + i] = row[i];
  }
  const SosSec<E> q = edge_section(a, b);
  const C na1 = up(q.na1), na2 = up(q.na2), c0 = up(q.c0), c1 = up(q.c1);
  const C det = C(1) - na1 - na2;  // det(I - A) = 1 + a1 + a2
  const E *x = a.x + b * a.T;
  const C u0 = up(a.e > 0 ? pad_front(x, a.T, a.e, a.mode, 0) : x[0]);
  // zi = (I - A)^-1 c with I - A = [[1 + a1, -1], [a2, 1]]
  C h0 = (c0 + c1) / det * u0;
  C h1 = (na2 * c0 + (C(1) - na1) * c1) / det * u0;
  for (int64_t j = 0; j < a.e; ++j) {
    const C u = up(pad_front(x, a.T, a.e, a.mode, j));
    const C n0 = na1 * h0 + h1 + c0 * u;
    h1 = na2 * h0 + c1 * u;
    h0 = n0;
  }
  a.state[b * 2] = down<E>(h0);
  a.state[b * 2 + 1] = down<E>(h1);
}

// Pass 2 entry state (adjoint coordinates, the REV cascade's grad_zf slot):
// the back pad stepped from pass 1's final state, its outputs y1b[j] folded
// as sum_j (A^T)^j e0 y1b[j] on top of (A^T)^e times the steady state of its
// last output (of y1[T-1] when e = 0).
template <typename E>
__global__ void filtfilt_mid_kernel(FiltfiltEdge<E> a) {
  using C = typename Wide<E>::type;
  const int64_t b = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= a.B) return;
  const SosSec<E> q = edge_section(a, b);
  const C b0 = up(q.b0), na1 = up(q.na1), na2 = up(q.na2), c0 = up(q.c0), c1 = up(q.c1);
  const C det = C(1) - na1 - na2;
  const E *x = a.x + b * a.T;
  C h0 = up(a.zf1[b * 2]), h1 = up(a.zf1[b * 2 + 1]);
  // P = (A^T)^j, A^T = [[-a1, -a2], [1, 0]]; acc = sum_j P e0 y1b[j]
  C p00 = C(1), p01 = C(0), p10 = C(0), p11 = C(1);
  C m0 = C(0), m1 = C(0);
  C y0 = a.e > 0 ? C(0) : up(a.y1[b * a.T + a.T - 1]);
  for (int64_t j = 0; j < a.e; ++j) {
    const C u = up(pad_back(x, a.T, a.mode, j));
    const C yb = h0 + b0 * u;
    m0 += p00 * yb;
    m1 += p10 * yb;
    const C n00 = na1 * p00 + na2 * p10, n01 = na1 * p01 + na2 * p11;
    p10 = p00;
    p11 = p01;
    p00 = n00;
    p01 = n01;
    const C n0 = na1 * h0 + h1 + c0 * u;
    h1 = na2 * h0 + c1 * u;
    h0 = n0;
    y0 = yb;
  }
  // m* = (I - A^T)^-1 e0 y0 = y0 / det (1, 1)
  const C s = y0 / det;
  m0 += (p00 + p01) * s;
  m1 += (p10 + p11) * s;
  a.state[b * 2] = down<E>(m0);
  a.state[b * 2 + 1] = down<E>(m1);
}

}  // namespace phs
