// Fused cascade of second-order sections (biquads), forward and adjoint, in
// one single-pass kernel per direction, for gfx950.
//
// Section s of row b has coefficients (b0, b1, b2, a1, a2) (a0 = 1) and runs
// the transposed direct form II of philtorch's lfilter(form="tdf2")
// (philtorch/lti/filtering.py:273-333 building state_space, lti/ssm.py:386-510):
//   y[t] = h[t-1].0 + b0 u[t],     h[t] = A h[t-1] + c u[t],
//   A = [[-a1, 1], [-a2, 0]],      c = (b1 - b0 a1, b2 - b0 a2),
// with h[-1] = zi[b, s] and zf[b, s] = h[T-1]; section s+1 filters section s's
// output.  The adjoint of the cascade is the transposed cascade, run backwards
// in time with the sections in reverse order:
//   mu[t] = A^T mu[t+1] + e0 g[t],   gu[t] = c . mu[t+1] + b0 g[t],
// where mu[t+1] = dL/dh[t], mu[T] = dL/dzf and mu[0] = dL/dzi.  It needs no
// forward values, so one kernel template serves both directions.
// Coefficient gradients pair mu with the forward input u and state h, which
// the backward recomputes inside its tile from x and the states the forward
// kernel checkpoints every kSosCkptEvery<E> steps: the entry state of every
// lane chunk of the backward, so the recompute runs each lane on its own.
//
// Per tile and section (tile layout as in phs_scan.hpp: data waves own
// contiguous segments of R rounds of 64*K steps; the backward mirrors waves,
// rounds and lanes in memory so that scan order is always ascending):
//   * pass 1: each lane folds its K steps from a zero state into the vector
//     part of an affine map; the matrix part is A^K for every lane, so a wave
//     scan of vector parts alone (DPP row shifts with the uniform multipliers
//     A^(K 2^j) inside 16-lane rows, then row totals with per-lane powers
//     of A^K computed once per section) gives each lane's exclusive prefix;
//   * the look-back wave combines the wave aggregates, publishes the tile's
//     aggregate of this section and resolves the section's entry state by
//     decoupled look-back over that section's own status row (the protocol,
//     tags and fallback of phs_scan.hpp);
//   * pass 2: every lane re-runs its steps from its exact entry state, and the
//     outputs replace the inputs in registers for the next section.
// Tile q's section s waits on tile q-1's section s, which in turn only needs
// tile q-1's sections below s: the dependence is a wavefront S sections deep,
// not a chain along the row.
#pragma once

#include "phs_scan.hpp"

namespace phs {

// Steps between forward state checkpoints: the gradient backward's lane
// chunk (fp32 32 steps, fp64 8), whose entry states the forward writes.
template <typename E>
constexpr int kSosCkptEvery = sizeof(E) == 4 ? 32 : 8;
constexpr int kSosMaxSections = 8;     // sections per launch (LDS of the gradient backward)

// The gradient backward needs every section's forward input inside its tile.
// Its forward recompute keeps in LDS the inputs of sections kept_step and
// 2 kept_step (those below S), so that re-deriving the input of section s
// runs only the sections from the nearest kept one below it: C4's eight
// sections with kept_step 3 take 7 section runs per tile instead of 28.
constexpr int kSosKeptSlots = 2;
__host__ __device__ constexpr int sos_kept_slots(int S, int step) {
  return step <= 0 ? 0 : (step < S ? 1 : 0) + (2 * step < S ? 1 : 0);
}

// Tile shape: W data waves plus one look-back wave; K steps per lane and
// round (a power of two dividing kSosCkptEvery<E>), R rounds (a power of
// two).
template <typename E, int K_, int R_, int W_>
struct SosShape {
  static constexpr int kWaves = W_;
  static constexpr int kThreads = 64 * (kWaves + 1);
  static constexpr int K = K_;
  static constexpr int R = R_;
  static constexpr int kWaveSeg = 64 * K * R;
  static constexpr int kTile = kWaves * kWaveSeg;
  static_assert(R >= 1 && (R & (R - 1)) == 0, "a power-of-two number of rounds");
  static_assert((K & (K - 1)) == 0 && kSosCkptEvery<E> % K == 0, "K must be a power of two dividing kSosCkptEvery");
  static_assert(kTile % kSosCkptEvery<E> == 0, "tiles start on checkpoints");
  static_assert((K * sizeof(E)) % 16 == 0, "chunks must be whole 16-byte vectors");
};

template <typename E>
struct SosArgs {
  using C = typename Wide<E>::type;
  const E *sos;            // [rows, S, 6]: b0 b1 b2 a0 a1 a2 (a0 = 1)
  int64_t sos_row_stride;  // elements between rows (0 = one set for all rows)
  // one biquad given as lfilter's b and a where they lie (S = 1; sos unused):
  // b [rows, nb] (nb <= 3, missing taps zero), a [rows, 2] (after the
  // leading 1), each row at its own stride (0 = shared)
  const E *fb, *fa;
  int64_t fb_row_stride, fa_row_stride;
  int nb;
  const E *in;             // forward: x;  backward: grad of y
  E *out;                  // forward: y;  backward: grad of x (nullable)
  const E *virt;           // forward: zi;  backward: grad of zf  ([B, S, 2], nullable = zeros)
  E *fin;                  // forward: zf;  backward: grad of zi  ([B, S, 2], nullable)
  Vec2<C> *ckpt;           // [B, S, n_ckpt] states entering every kSosCkptEvery-th step:
                           // written forward (nullable), read by the gradient backward
  const E *x;              // gradient backward: the forward input
  C *partials;             // gradient backward: [B, S, tiles, kWaves, 5] coefficient sums
  int64_t B, T_len, tiles_per_row, n_ckpt;
  int S;
  uint64_t b_magic;            // tile id -> row by multiply and shift (row_split)
  unsigned b_shift;
  unsigned long long *claims;  // kStripes claim words (workspace offset 0)
  unsigned tiles;              // B * tiles_per_row
  unsigned per_stripe;         // claims per stripe (grid = per_stripe * kStripes)
  unsigned spin_limit;         // look-back polls before the self-compute fallback
  unsigned agg_only;           // testing: tiles after a row's first publish no inclusive state
  uint64_t *status;            // [B, S, tiles, kStride] status words of this call
  int vec_ok;
  int kept_step;               // gradient backward: sections whose input stays in LDS (0: none)
  int out_lds;                 // gradient backward: kept slot 0 holds the output's LDS transpose
};

// One section, in the form the steps use.
template <typename E>
struct SosSec {
  E b0, c0, c1, na1, na2;  // c = b[1:] - b0 a;  na = -a
};

// Coefficients (b0, b1, b2, a1, a2) of section s of row r.
template <typename E>
struct SosCoef {
  E b0, b1, b2, a1, a2;
};

template <typename E>
__device__ __forceinline__ SosCoef<E> sec_coef(const SosArgs<E> &a, int64_t r, int s) {
  if (a.fb) {
    const E *pb = a.fb + r * a.fb_row_stride, *pa = a.fa + r * a.fa_row_stride;
    return {pb[0], a.nb > 1 ? pb[1] : E(0), a.nb > 2 ? pb[2] : E(0), pa[0], pa[1]};
  }
  const E *p = a.sos + r * a.sos_row_stride + 6 * s;
  return {p[0], p[1], p[2], p[4], p[5]};
}

template <typename E>
__device__ __forceinline__ SosSec<E> load_sec(const SosArgs<E> &a, int64_t r, int s) {
  const SosCoef<E> k = sec_coef(a, r, s);
  return {k.b0, k.b1 - k.b0 * k.a1, k.b2 - k.b0 * k.a2, -k.a1, -k.a2};
}

// Section matrix A in compute precision.
template <typename E>
__device__ __forceinline__ Mat2<typename Wide<E>::type> sec_matrix(const SosSec<E> &q) {
  using C = typename Wide<E>::type;
  return {up(q.na1), C(1), up(q.na2), C(0)};
}

// P[0] = A^K, P[j] = A^(K 2^j).
template <typename E, int K, int NP>
__device__ __forceinline__ void sec_powers(const Mat2<typename Wide<E>::type> &A,
                                           Mat2<typename Wide<E>::type> (&P)[NP]) {
  using Alg = Block2<E>;
  Mat2<typename Wide<E>::type> m = A;
#pragma unroll
  for (int k = 1; k < K; k <<= 1) m = Alg::cmul(m, m);
  P[0] = m;
#pragma unroll
  for (int j = 1; j < NP; ++j) P[j] = Alg::cmul(P[j - 1], P[j - 1]);
}

// A^(K cnt) for cnt in [0, 64), from P (powers of one matrix commute).
template <typename E, int NP>
__device__ __forceinline__ Mat2<typename Wide<E>::type> lane_power(const Mat2<typename Wide<E>::type> (&P)[NP],
                                                                   int cnt) {
  using Alg = Block2<E>;
  Mat2<typename Wide<E>::type> r = Alg::cone();
#pragma unroll
  for (int j = 0; j < 6; ++j)
    if ((cnt >> j) & 1) r = Alg::cmul(P[j], r);
  return r;
}

// Powers of one section's matrix, built by one wave into LDS once per tile
// and section: pw[n] = A^(K n) for n = 0..64, and seg = A^(64 K R), the
// matrix part of a whole wave segment.  Every multiplier the lane scans need
// is one of them, and their transposes serve the adjoint ((A^T)^n = (A^n)^T).
template <typename C>
struct SecPowers {
  Mat2<C> pw[65];
  Mat2<C> seg;
};

// W > 0: also wm[j] = seg^j for j = 0..W (the matrix parts of the tile's
// wave prefixes; wm[W] is the tile matrix).
template <typename E, int K, int R, int W = 0>
__device__ __forceinline__ void build_powers(SecPowers<typename Wide<E>::type> *t, const SosSec<E> &q, int lane,
                                             Mat2<typename Wide<E>::type> *wm = nullptr) {
  using Alg = Block2<E>;
  using Mt = Mat2<typename Wide<E>::type>;
  Mt P[7];
  sec_powers<E, K, 7>(sec_matrix(q), P);
  t->pw[lane] = lane_power<E, 7>(P, lane);
  Mt seg = P[6];
#pragma unroll
  for (int r = 1; r < R; r <<= 1) seg = Alg::cmul(seg, seg);
  if (lane == 0) {
    t->pw[64] = P[6];
    t->seg = seg;
  }
  if constexpr (W > 0) {
    static_assert(W < 64, "one lane per power");
    Mt m = Alg::cone();
#pragma unroll
    for (int j = 0; j < W; ++j) {
      if (lane == j) wm[j] = m;
      m = Alg::cmul(seg, m);
    }
    if (lane == W) wm[W] = m;
  }
}

// A o + x (TR: A^T o + x)
template <bool TR, typename C>
__device__ __forceinline__ Vec2<C> mva(const Mat2<C> &A, const Vec2<C> &o, const Vec2<C> &x) {
  if constexpr (TR)
    return {mad(A.m00, o.v0, mad(A.m10, o.v1, x.v0)), mad(A.m01, o.v0, mad(A.m11, o.v1, x.v1))};
  else
    return {mad(A.m00, o.v0, mad(A.m01, o.v1, x.v0)), mad(A.m10, o.v0, mad(A.m11, o.v1, x.v1))};
}

template <bool TR, typename C>
__device__ __forceinline__ Mat2<C> maybe_transpose(const Mat2<C> &A) {
  if constexpr (TR)
    return {A.m00, A.m10, A.m01, A.m11};
  else
    return A;
}

constexpr int kDppRowShl1 = 0x101, kDppRowShl2 = 0x102, kDppRowShl4 = 0x104, kDppRowShl8 = 0x108;
constexpr int kDppWaveShl1 = 0x130;

// Inclusive scans of the vector parts of maps (B^K, v[n]) over the wave, for
// N independent values at once (their latency chains interleave), lane 0
// first (UP) or lane 63 first (!UP), B = A (TR: A^T), multipliers from t:
// v_i <- v_i + B^(K d) v_(i -+ d) for d = 1, 2, 4, 8 inside each 16-lane row
// (DPP row shifts); a lane at row position r then holds its row's prefix up
// to itself (UP) or suffix from itself (!UP), and adds the preceding row's
// total, r+1 (UP) or 16-r (!UP) lanes away, then that of the preceding pair
// of rows (UP: DPP row_bcast 15/31; !UP: bpermute from the mirrored lanes).
template <bool UP, bool TR, typename C, int N>
__device__ __forceinline__ void lti_scan(Vec2<C> (&v)[N], int lane, const SecPowers<C> &t) {
  const int r = lane & 15;
  Vec2<C> o[N];
#define PHS_SOS_LEVEL(CTRL_UP, CTRL_DOWN, COND_UP, COND_DOWN, MAT)            \
  {                                                                           \
    _Pragma("unroll") for (int n = 0; n < N; ++n) o[n] = dpp_move<UP ? CTRL_UP : CTRL_DOWN, 0xF>(v[n]); \
    if (UP ? (COND_UP) : (COND_DOWN)) {                                       \
      const Mat2<C> m = (MAT);                                                \
      _Pragma("unroll") for (int n = 0; n < N; ++n) v[n] = mva<TR>(m, o[n], v[n]); \
    }                                                                         \
  }
  PHS_SOS_LEVEL(kDppRowShr1, kDppRowShl1, r >= 1, r <= 14, t.pw[1])
  PHS_SOS_LEVEL(kDppRowShr2, kDppRowShl2, r >= 2, r <= 13, t.pw[2])
  PHS_SOS_LEVEL(kDppRowShr4, kDppRowShl4, r >= 4, r <= 11, t.pw[4])
  PHS_SOS_LEVEL(kDppRowShr8, kDppRowShl8, r >= 8, r <= 7, t.pw[8])
#undef PHS_SOS_LEVEL
  if constexpr (UP) {
    const Mat2<C> m1 = t.pw[r + 1], m2 = t.pw[(lane & 31) + 1];
#pragma unroll
    for (int n = 0; n < N; ++n) o[n] = dpp_move<kDppRowBcast15, 0xA>(v[n]);
    if (lane & 16)
#pragma unroll
      for (int n = 0; n < N; ++n) v[n] = mva<TR>(m1, o[n], v[n]);
#pragma unroll
    for (int n = 0; n < N; ++n) o[n] = dpp_move<kDppRowBcast31, 0xC>(v[n]);
    if (lane >= 32)
#pragma unroll
      for (int n = 0; n < N; ++n) v[n] = mva<TR>(m2, o[n], v[n]);
  } else {
    const Mat2<C> m1 = t.pw[16 - r], m2 = t.pw[32 - (lane & 31)];
#pragma unroll
    for (int n = 0; n < N; ++n) o[n] = shfl_from(v[n], ((lane | 15) + 1) & 63);
    if ((lane & 16) == 0)
#pragma unroll
      for (int n = 0; n < N; ++n) v[n] = mva<TR>(m1, o[n], v[n]);
#pragma unroll
    for (int n = 0; n < N; ++n) o[n] = shfl_from(v[n], 32);
    if (lane < 32)
#pragma unroll
      for (int n = 0; n < N; ++n) v[n] = mva<TR>(m2, o[n], v[n]);
  }
}

// Value of the previous lane in scan order (the first lane gets `first`).
template <bool UP, typename X>
__device__ __forceinline__ X lane_prev(const X &v, int lane, const X &first) {
  X o = dpp_move<UP ? kDppWaveShr1 : kDppWaveShl1, 0xF>(v);
  return (UP ? lane == 0 : lane == 63) ? first : o;
}

// ------------------------------------------------------------ lane steps
// Forward fold of steps [t0, t0+K) from a zero state (pass 1).  Steps past the
// row end read zero inputs and follow every valid step: they only change
// states nobody reads.
template <typename E, int K>
__device__ __forceinline__ Vec2<typename Wide<E>::type> fold_fwd(const SosSec<E> &q, const E (&u)[K]) {
  E v0 = E(0), v1 = E(0);
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const E x = u[k];
    const E n0 = fma(q.na1, v0, fma(q.c0, x, v1));
    v1 = fma(q.na2, v0, q.c1 * x);
    v0 = n0;
  }
  return {up(v0), up(v1)};
}

// Forward run of steps [t0, t0+K) from state h (pass 2): outputs replace the
// inputs, zero past the row end; zf (nullable) receives h[T-1].
template <typename E, int K>
__device__ __forceinline__ void run_fwd(const SosSec<E> &q, Vec2<E> h, E (&u)[K], int64_t t0, int64_t T, E *zf) {
  if (t0 + K <= T) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const E x = u[k];
      u[k] = fma(q.b0, x, h.v0);
      const E n0 = fma(q.na1, h.v0, fma(q.c0, x, h.v1));
      h.v1 = fma(q.na2, h.v0, q.c1 * x);
      h.v0 = n0;
    }
    if (zf && t0 + K == T) {
      zf[0] = h.v0;
      zf[1] = h.v1;
    }
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const E x = u[k];
      if (t0 + k < T) {
        u[k] = fma(q.b0, x, h.v0);
        const E n0 = fma(q.na1, h.v0, fma(q.c0, x, h.v1));
        h.v1 = fma(q.na2, h.v0, q.c1 * x);
        h.v0 = n0;
        if (zf && t0 + k == T - 1) {
          zf[0] = h.v0;
          zf[1] = h.v1;
        }
      } else {
        u[k] = E(0);
      }
    }
  }
}

// Adjoint fold of steps t0+K-1 down to t0 from a zero state.  Past the row end
// the gradient is zero; the step at t = T (present when the row does not end on
// a tile boundary) injects dL/dzf, so that mu[T] = dL/dzf exactly.
template <typename E, int K>
__device__ __forceinline__ Vec2<typename Wide<E>::type> fold_adj(const SosSec<E> &q, const E (&g)[K], int64_t t0,
                                                                 int64_t T, const Vec2<E> &gzf) {
  E m0 = E(0), m1 = E(0);
  if (t0 + K <= T) {
#pragma unroll
    for (int kk = 0; kk < K; ++kk) {
      const int k = K - 1 - kk;
      const E n0 = fma(q.na1, m0, fma(q.na2, m1, g[k]));
      m1 = m0;
      m0 = n0;
    }
  } else {
#pragma unroll
    for (int kk = 0; kk < K; ++kk) {
      const int k = K - 1 - kk;
      const int64_t t = t0 + k;
      if (t < T) {
        const E n0 = fma(q.na1, m0, fma(q.na2, m1, g[k]));
        m1 = m0;
        m0 = n0;
      } else if (t == T) {
        m0 = gzf.v0;
        m1 = gzf.v1;
      }
    }
  }
  return {up(m0), up(m1)};
}

// Coefficient-gradient sums of one section (per lane, then per wave):
// a1: sum mu0 h0,  a2: sum mu1 h0,  c0: sum mu0 u,  c1: sum mu1 u,  b0: sum g u,
// with mu = mu[t+1] = dL/dh[t], h0 = h[t-1].0 = y[t] - b0 u[t].
template <typename C>
struct SosAcc {
  C a1, a2, c0, c1, b0;
};

// Adjoint run of steps t0+K-1 down to t0 from mu (pass 2): grad of the
// section input replaces g (zero past the row end); gzi (nullable) receives
// mu[0].  With GRAD, u/y are the forward input and output of the section and
// the sums go to acc.
template <typename E, int K, bool GRAD>
__device__ __forceinline__ void run_adj(const SosSec<E> &q, Vec2<E> mu, E (&g)[K], int64_t t0, int64_t T,
                                        const Vec2<E> &gzf, E *gzi, const E (&u)[GRAD ? K : 1],
                                        const E (&y)[GRAD ? K : 1], SosAcc<E> &acc) {
  auto step = [&](int k) {
    const E gk = g[k];
    if constexpr (GRAD) {
      const E uk = u[k];
      const E h0 = fma(-q.b0, uk, y[k]);
      acc.a1 = fma(mu.v0, h0, acc.a1);
      acc.a2 = fma(mu.v1, h0, acc.a2);
      acc.c0 = fma(mu.v0, uk, acc.c0);
      acc.c1 = fma(mu.v1, uk, acc.c1);
      acc.b0 = fma(gk, uk, acc.b0);
    }
    g[k] = fma(q.c0, mu.v0, fma(q.c1, mu.v1, q.b0 * gk));
    const E n0 = fma(q.na1, mu.v0, fma(q.na2, mu.v1, gk));
    mu.v1 = mu.v0;
    mu.v0 = n0;
  };
  if (t0 + K <= T) {
#pragma unroll
    for (int kk = 0; kk < K; ++kk) step(K - 1 - kk);
  } else {
#pragma unroll
    for (int kk = 0; kk < K; ++kk) {
      const int k = K - 1 - kk;
      const int64_t t = t0 + k;
      if (t < T) {
        step(k);
      } else {
        if (t == T) mu = gzf;
        g[k] = E(0);
      }
    }
  }
  if (gzi && t0 == 0) {
    gzi[0] = mu.v0;
    gzi[1] = mu.v1;
  }
}

// The same over N chunks of one lane at once (independent chains, so their
// latencies overlap); chunk n starts at t0[n].  Only when a chunk reaches past
// the row end does a chunk take the single-chunk path with its bounds checks.
template <typename E, int K, int N>
__device__ __forceinline__ bool chunks_full(const int64_t (&t0)[N], int64_t T) {
  bool full = true;
#pragma unroll
  for (int n = 0; n < N; ++n) full = full && t0[n] + K <= T;
  return full;
}

template <typename E, int K, int N>
__device__ __forceinline__ void fold_fwd_n(const SosSec<E> &q, const E (&u)[N][K],
                                           Vec2<typename Wide<E>::type> (&out)[N]) {
  E v0[N], v1[N];
#pragma unroll
  for (int n = 0; n < N; ++n) v0[n] = v1[n] = E(0);
#pragma unroll
  for (int k = 0; k < K; ++k)
#pragma unroll
    for (int n = 0; n < N; ++n) {
      const E x = u[n][k];
      const E n0 = fma(q.na1, v0[n], fma(q.c0, x, v1[n]));
      v1[n] = fma(q.na2, v0[n], q.c1 * x);
      v0[n] = n0;
    }
#pragma unroll
  for (int n = 0; n < N; ++n) out[n] = {up(v0[n]), up(v1[n])};
}

template <typename E, int K, int N>
__device__ __forceinline__ void run_fwd_n(const SosSec<E> &q, Vec2<E> (&h)[N], E (&u)[N][K],
                                          const int64_t (&t0)[N], int64_t T, E *zf) {
  if (chunks_full<E, K, N>(t0, T)) {
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
      for (int n = 0; n < N; ++n) {
        const E x = u[n][k];
        u[n][k] = fma(q.b0, x, h[n].v0);
        const E n0 = fma(q.na1, h[n].v0, fma(q.c0, x, h[n].v1));
        h[n].v1 = fma(q.na2, h[n].v0, q.c1 * x);
        h[n].v0 = n0;
      }
    if (zf)
#pragma unroll
      for (int n = 0; n < N; ++n)
        if (t0[n] + K == T) {
          zf[0] = h[n].v0;
          zf[1] = h[n].v1;
        }
  } else {
#pragma unroll
    for (int n = 0; n < N; ++n) run_fwd<E, K>(q, h[n], u[n], t0[n], T, zf);
  }
}

template <typename E, int K, int N>
__device__ __forceinline__ void fold_adj_n(const SosSec<E> &q, const E (&g)[N][K], const int64_t (&t0)[N],
                                           int64_t T, const Vec2<E> &gzf, Vec2<typename Wide<E>::type> (&out)[N]) {
  if (chunks_full<E, K, N>(t0, T)) {
    E m0[N], m1[N];
#pragma unroll
    for (int n = 0; n < N; ++n) m0[n] = m1[n] = E(0);
#pragma unroll
    for (int kk = 0; kk < K; ++kk)
#pragma unroll
      for (int n = 0; n < N; ++n) {
        const E n0 = fma(q.na1, m0[n], fma(q.na2, m1[n], g[n][K - 1 - kk]));
        m1[n] = m0[n];
        m0[n] = n0;
      }
#pragma unroll
    for (int n = 0; n < N; ++n) out[n] = {up(m0[n]), up(m1[n])};
  } else {
#pragma unroll
    for (int n = 0; n < N; ++n) out[n] = fold_adj<E, K>(q, g[n], t0[n], T, gzf);
  }
}

template <typename E, int K, int N, bool GRAD>
__device__ __forceinline__ void run_adj_n(const SosSec<E> &q, Vec2<E> (&mu)[N], E (&g)[N][K],
                                          const int64_t (&t0)[N], int64_t T, const Vec2<E> &gzf, E *gzi,
                                          const E (&u)[GRAD ? N : 1][GRAD ? K : 1],
                                          const E (&y)[GRAD ? N : 1][GRAD ? K : 1], SosAcc<E> (&acc)[N]) {
  if (chunks_full<E, K, N>(t0, T)) {
#pragma unroll
    for (int kk = 0; kk < K; ++kk)
#pragma unroll
      for (int n = 0; n < N; ++n) {
        const int k = K - 1 - kk;
        const E gk = g[n][k];
        if constexpr (GRAD) {
          const E uk = u[n][k];
          const E h0 = fma(-q.b0, uk, y[n][k]);
          acc[n].a1 = fma(mu[n].v0, h0, acc[n].a1);
          acc[n].a2 = fma(mu[n].v1, h0, acc[n].a2);
          acc[n].c0 = fma(mu[n].v0, uk, acc[n].c0);
          acc[n].c1 = fma(mu[n].v1, uk, acc[n].c1);
          acc[n].b0 = fma(gk, uk, acc[n].b0);
        }
        g[n][k] = fma(q.c0, mu[n].v0, fma(q.c1, mu[n].v1, q.b0 * gk));
        const E n0 = fma(q.na1, mu[n].v0, fma(q.na2, mu[n].v1, gk));
        mu[n].v1 = mu[n].v0;
        mu[n].v0 = n0;
      }
    if (gzi)
#pragma unroll
      for (int n = 0; n < N; ++n)
        if (t0[n] == 0) {
          gzi[0] = mu[n].v0;
          gzi[1] = mu[n].v1;
        }
  } else {
#pragma unroll
    for (int n = 0; n < N; ++n) run_adj<E, K, GRAD>(q, mu[n], g[n], t0[n], T, gzf, gzi, u[GRAD ? n : 0], y[GRAD ? n : 0], acc[n]);
  }
}

template <typename E>
__device__ __forceinline__ Vec2<E> load_pair(const E *p, bool valid) {
  return valid ? Vec2<E>{p[0], p[1]} : Vec2<E>{E(0), E(0)};
}

// ------------------------------------------------------------ look-back
// Every tile aggregate of an LTI section has the same matrix part, the tile
// matrix G = B^(tile steps) (B = A forward, A^T for the adjoint), so a status
// entry carries vectors only: the inclusive state (words 0-3) and the tile's
// zero-entry aggregate (words 4-7), each 32-bit chunk a tagged 64-bit word as
// in phs_scan.hpp.  With lane i looking at tile q-1-i and k the first lane
// holding an inclusive state,
//   state entering tile q = sum_{i<k} G^i agg(q-1-i) + G^k inc(q-1-k),
// one matrix-vector product per lane and a wave sum.  The first window holds
// the kSosLookFirst nearest tiles (the inclusive state is almost always among
// them), further windows 64; a window's sum is weighted by G^(tiles passed).
constexpr int kSosLookFirst = 8;
constexpr int kSosStatusWords = 8;
constexpr int kSosLookPitch = kSosStatusWords + 1;  // odd LDS pitch: no bank conflicts
constexpr int kSosLookWords = 64 * kSosLookPitch;

// Tile-level powers for one section: gl = G^lane, gfirst = G^kSosLookFirst and
// g64 = G^64 (the weights of the windows passed).
template <typename C>
struct TilePowers {
  Mat2<C> gl, gfirst, g64;
};

template <typename E>
__device__ __forceinline__ TilePowers<typename Wide<E>::type> tile_powers(const Mat2<typename Wide<E>::type> &G,
                                                                         int lane) {
  using Alg = Block2<E>;
  Mat2<typename Wide<E>::type> g[7];
  g[0] = G;
#pragma unroll
  for (int j = 1; j < 7; ++j) g[j] = Alg::cmul(g[j - 1], g[j - 1]);
  static_assert(kSosLookFirst == 8, "gfirst is G^8");
  return {lane_power<E, 7>(g, lane), g[3], g[6]};
}

// One section's look-back for tile q of a row: polls until the entry state is
// known (true, in `out`) or `spin_limit` polls found a predecessor still
// unpublished (false).  `virt` is the state before the row's first tile.
template <typename E>
__device__ bool sos_lookback(const uint64_t *row_status, const Vec2<typename Wide<E>::type> &virt, int lane,
                             unsigned tag, unsigned spin_limit, uint64_t *s_look,
                             const TilePowers<typename Wide<E>::type> &tp, int64_t q,
                             Vec2<typename Wide<E>::type> &out) {
  using Alg = Block2<E>;
  using C = typename Wide<E>::type;
  using V = Vec2<C>;
  constexpr int kS = kSosStatusWords, kP = kSosLookPitch;
  V acc = Alg::szero();
  Mat2<C> gm = Alg::cone();
  int64_t base = q - 1;
  unsigned polls = 0;
  int span = kSosLookFirst;
  auto add = [](const V &p, const V &o) -> V { return {p.v0 + o.v0, p.v1 + o.v1}; };
  while (true) {
    const int n = base + 1 > span ? span : int(base + 1);  // tiles in the window
    const uint64_t *win = row_status + (base + 1 - n) * kS + lane;
    uint64_t words[kS];
#pragma unroll
    for (int i = 0; i < kS; ++i) {
      words[i] = 0;
      if (i * 64 + lane < n * kS)  // word i*64+lane of the window
        words[i] = __hip_atomic_load(win + i * 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int i = 0; i < kS; ++i) {
      const int j = i * 64 + lane;
      s_look[(j / kS) * kP + (j % kS)] = words[i];
    }
    wave_sync();
    const int64_t p = base - lane;  // lane < n: window entry n-1-lane
    V inc = Alg::szero(), agg = Alg::szero();
    int st = 3;  // outside the window: no contribution, never inclusive
    if (lane < n) {
      const uint64_t *e = s_look + (n - 1 - lane) * kP;
      const bool inc_ok = unpack(e, inc, tag);
      const bool agg_ok = unpack(e + 4, agg, tag);
      st = inc_ok ? 2 : (agg_ok ? 1 : 0);
    } else if (p == -1) {
      st = 2;
      inc = virt;
    }
    wave_sync();
    const uint64_t incm = __ballot(st == 2);
    const int k = incm ? __builtin_ctzll(incm) : 64;
    const uint64_t low = (k >= 64) ? ~0ull : ((1ull << k) - 1ull);
    if (__ballot(st == 0) & low) {
      if (++polls >= spin_limit) return false;
      __builtin_amdgcn_s_sleep(1);
      continue;
    }
    V c = Alg::szero();
    if (lane < k && lane < n) c = Alg::affine(tp.gl, agg, Alg::szero());
    if (lane == k) c = Alg::affine(tp.gl, inc, Alg::szero());
    const V sum = read_lane(wave_scan_incl(c, lane, add), 63);
    acc = Alg::affine(gm, sum, acc);
    if (k < 64) {
      out = acc;
      return true;
    }
    gm = Alg::cmul(n == 64 ? tp.g64 : tp.gfirst, gm);
    base -= n;
    span = 64;
  }
}

// ------------------------------------------------------------ look-back fallback
// State entering scan positions [span, ...) of section s_target in row b,
// computed by one wave straight from the inputs: the cascade (forward) or the
// adjoint cascade (REV) over the whole row prefix in scan order, 64*K steps
// per iteration (K = 4 whatever the tile's lane chunk: the kernel's VGPR
// count is the largest of its own and its callees', and at the tile's K this
// function set it, 229 against 111 for the fp32 backward), every section up
// to s_target carrying its state across iterations.  `lds` (the look-back
// staging area, free by then) holds the carries and the section's powers.
// Taken only when predecessors did not publish within the poll budget.  The
// arguments come by value: a reference would make every thread of the kernel
// keep a private copy of them.
template <typename E, class Sh, bool REV>
__device__ __noinline__ Vec2<typename Wide<E>::type> sos_prefix_fallback(const SosArgs<E> a, int64_t b,
                                                                        int s_target, int64_t span, int lane,
                                                                        uint64_t *lds) {
  using Alg = Block2<E>;
  using C = typename Wide<E>::type;
  using V = Vec2<C>;
  constexpr int K = Sh::K < 4 ? Sh::K : 4;
  static_assert(Sh::kTile % (64 * K) == 0, "tiles are whole fallback iterations");
  V *carry = reinterpret_cast<V *>(lds);
  SecPowers<C> *tab = reinterpret_cast<SecPowers<C> *>(lds + kSosMaxSections * (sizeof(V) / sizeof(uint64_t)));
  const int S = a.S;
  const int64_t T = a.T_len;
  const int64_t row_end = a.tiles_per_row * Sh::kTile;
  const int n = REV ? S - s_target : s_target + 1;  // sections in processing order
  const E *inrow = a.in + b * T;
  const bool row_virt = !REV || (T % Sh::kTile) == 0;
  wave_sync();
  if (lane == 0)
    for (int i = 0; i < n; ++i) {
      const int s = REV ? S - 1 - i : i;
      const Vec2<E> v = load_pair(a.virt + (b * S + s) * 2, a.virt != nullptr && row_virt);
      carry[i] = {up(v.v0), up(v.v1)};
    }
  wave_sync();
  const E zero = E(0);
  const SosAcc<E> none{};
  for (int64_t off = 0; off < span; off += 64 * K) {
    const int64_t t0 = REV ? row_end - off - int64_t(lane + 1) * K : off + int64_t(lane) * K;
    const int64_t t0s[1] = {t0};
    E u[1][K];
    load_chunk<E, K>(inrow, t0, T, a.vec_ok != 0, u[0], zero);
    for (int i = 0; i < n; ++i) {
      const int s = REV ? S - 1 - i : i;
      const SosSec<E> q = load_sec(a, b, s);
      wave_sync();
      build_powers<E, K, Sh::R>(tab, q, lane);
      wave_sync();
      const Vec2<E> gzf = load_pair(a.virt + (b * S + s) * 2, REV && a.virt != nullptr);
      V v[1];
      if constexpr (REV)
        fold_adj_n<E, K, 1>(q, u, t0s, T, gzf, v);
      else
        fold_fwd_n<E, K, 1>(q, u, v);
      lti_scan<true, REV>(v, lane, *tab);
      const V tot = read_lane(v[0], 63);
      const V ex = lane_prev<true>(v[0], lane, Alg::szero());
      const V c = carry[i];
      Vec2<E> h[1] = {Alg::store_s(mva<REV>(tab->pw[lane], c, ex))};
      const V cn = mva<REV>(tab->pw[64], c, tot);
      if constexpr (REV) {
        SosAcc<E> acc[1] = {none};
        const E unused[1][1] = {{zero}};
        run_adj_n<E, K, 1, false>(q, h, u, t0s, T, gzf, nullptr, unused, unused, acc);
      } else {
        run_fwd_n<E, K, 1>(q, h, u, t0s, T, nullptr);
      }
      wave_sync();
      if (lane == 0) carry[i] = cn;
      wave_sync();
    }
  }
  const V out = carry[n - 1];
  wave_sync();
  return out;
}

// ------------------------------------------------------------ the kernel
// REV : adjoint cascade (backward); GRAD: also the coefficient gradients
// (backward only: recomputes the forward inside the tile from a.x and a.ckpt).
//
// The tile visits its sections in order (backward: in reverse order, after,
// with GRAD, a recompute of the forward cascade that every lane runs on its
// own from its checkpointed entry states).  The look-back wave builds each
// visit's matrix powers two visits ahead into one of three LDS buffers
// (keeping the data waves' registers free of matrices) and resolves each
// section's entry state.  Barriers: powers of the first two visits; two per
// visit (wave aggregates ready, entry state ready).
// Waves per SIMD the launch bounds ask for: the fp32 forward 4 (128 VGPRs,
// a 15-wave tile and its look-back wave fill a CU), the fp32 backward 3 (168
// VGPRs: three workgroups per CU, so C4's 1264 backward tiles run in two
// generations instead of three); fp64 keeps its registers.
template <typename E, bool REV>
constexpr int kSosMinWaves = sizeof(E) == 4 ? (REV ? 3 : 4) : 1;

// Workgroups of shape Sh a CU holds at those bounds (four SIMDs).
template <typename E, class Sh, bool REV>
constexpr int kSosWgsPerCu = sizeof(E) == 4 ? 4 * kSosMinWaves<E, REV> / (Sh::kThreads / 64) : 1;

// ONE (gradient backward of a single section, the biquad op's, with the
// output's LDS slot): the prologue's load of x also goes to that slot, and
// the one visit reads its section's input from there instead of loading x a
// second time (the slot takes the output's transpose only after the visit
// has read it).  Holding x in registers instead spilled 124 VGPRs: it lives
// across the visit's fold and scan, where its input does not.
template <typename E, class Sh, bool REV, bool GRAD, bool ONE = false>
__global__ __launch_bounds__(Sh::kThreads, (kSosMinWaves<E, REV>)) void sos_kernel(SosArgs<E> a) {
  using Alg = Block2<E>;
  using C = typename Wide<E>::type;
  using V = Vec2<C>;
  using M = Map<Alg>;
  using SV = Vec2<E>;
  constexpr int K = Sh::K, R = Sh::R, W = Sh::kWaves;
  using Mt = Mat2<C>;
  static_assert(!GRAD || REV, "coefficient gradients come with the backward");
  static_assert(!ONE || GRAD, "the single-section form is the gradient backward's");

  __shared__ M s_wagg[W];
  __shared__ M s_wpre[W];
  __shared__ V s_in;
  __shared__ unsigned s_id, s_tag;
  __shared__ uint64_t s_look[kSosLookWords];
  __shared__ SecPowers<C> s_pow[3];
  // wide tiles: seg^j (j <= W) in LDS beside s_pow, built with it; narrow
  // ones keep the W + 1 matrices in the look-back wave's registers
  constexpr bool kWmatLds = W > 4;
  constexpr int kWm = kWmatLds ? W : 0;
  __shared__ Mt s_wmat[3][kWm + 1];
  // GRAD: lane entry states [S][W][R][64], then the kept sections' inputs
  // [slot][W][R][K][64] (slot i: section (i + 1) kept_step)
  extern __shared__ __align__(16) unsigned char sos_dyn[];
  SV *s_laneh = reinterpret_cast<SV *>(sos_dyn);
  E *s_uin = reinterpret_cast<E *>(sos_dyn + size_t(a.S) * W * R * 64 * sizeof(SV));
  // Whole rounds of the output leave through a lane-blocked LDS buffer of
  // the wave as 1 KB rows (lds_flush): static for the forward and the plain
  // backward; the gradient backward reuses the wave's part of kept slot 0
  // (a.out_lds), whose inputs are dead by then
  constexpr bool kOutLds = kLdsBlocked<E, K>;
  constexpr int kNVo = kOutLds ? int(K * sizeof(E) / 16) : 1;
  __shared__ uint4 s_out[(kOutLds && !GRAD) ? W * 64 * kNVo : 1];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the tile is the workgroup's index (dispatch order puts a tile's row
  // predecessors first); the look-back wave claims for the call's tag
  // (claim_tag), so the data waves' loads do not wait for the claim
  const int64_t id = blockIdx.x;
  if (id >= a.tiles) {  // padding of the last stripe round: counted, then gone
    if (tid == 0) claim_tile(a.claims, a.per_stripe, s_id, s_tag);
    return;
  }
  unsigned tag = 0;
  int64_t qs, b;  // position in scan order, row
  split_tile(id, a.B, a.b_magic, a.b_shift, qs, b);
  const int64_t tiles = a.tiles_per_row;
  const int64_t qf = REV ? tiles - 1 - qs : qs;  // position along time
  const int64_t T = a.T_len;
  const int S = a.S;
  const bool vec = a.vec_ok != 0;
  // the row's state before its first step in scan order; backward it is
  // dL/dzf only when no padded step t = T carries it
  const bool row_virt = !REV || (T % Sh::kTile) == 0;
  // visit v -> section: forward 0..S-1; backward S-1..0
  const int nvis = S;
  auto vis_sec = [S](int v) { return REV ? S - 1 - v : v; };

  if (w == W) {
    // ================= look-back wave
    build_powers<E, K, R, kWm>(&s_pow[0], load_sec(a, b, vis_sec(0)), lane, s_wmat[0]);
    if (nvis > 1) build_powers<E, K, R, kWm>(&s_pow[1], load_sec(a, b, vis_sec(1)), lane, s_wmat[1]);
    __syncthreads();  // powers of the first two visits
    tag = claim_tag(a.claims, a.per_stripe, lane);
    for (int v = 0; v < nvis; ++v) {
      const int s = vis_sec(v);
      uint64_t *row_status = a.status + ((b * S + s) * tiles) * kSosStatusWords;
      const SV vs = load_pair(a.virt + (b * S + s) * 2, a.virt != nullptr && row_virt);
      const V virt = {up(vs.v0), up(vs.v1)};
      // matrices of this section, before the aggregates are in: one wave
      // segment (Mw), the tile matrix G = Mw^W and G's powers
      const Mt Mw = maybe_transpose<REV>(s_pow[v % 3].seg);
      Mt Mp[kWmatLds ? 1 : W + 1];
      Mp[0] = Alg::cone();
      if constexpr (!kWmatLds) {
#pragma unroll
        for (int j = 1; j <= W; ++j) Mp[j] = Alg::cmul(Mw, Mp[j - 1]);
      }
      const Mt G = kWmatLds ? maybe_transpose<REV>(s_wmat[v % 3][W]) : Mp[kWmatLds ? 0 : W];
      const TilePowers<C> tp = tile_powers<E>(G, lane);
      // (polling for the predecessors before the aggregates are in measured
      // slower: a tile's predecessors reach each section about when it does)
      V yin = virt;
      __syncthreads();  // wave aggregates are in s_wagg
      // exclusive wave prefixes and the tile aggregate: every wave aggregate
      // has the matrix part Mw
      V pv = Alg::szero();
#pragma unroll
      for (int j = 0; j < W; ++j) {
        if (lane == 0) s_wpre[j] = M{kWmatLds ? maybe_transpose<REV>(s_wmat[v % 3][j]) : Mp[kWmatLds ? 0 : j], pv};
        pv = Alg::affine(Mw, pv, s_wagg[j].x);
      }
      if (qs > 0) {
        if (lane == 0) publish(row_status + qs * kSosStatusWords + 4, pv, tag);
        if (!sos_lookback<E>(row_status, virt, lane, tag, a.spin_limit, s_look, tp, qs, yin))
          yin = sos_prefix_fallback<E, Sh, REV>(a, b, s, qs * Sh::kTile, lane, s_look);
      }
      if (qs + 1 < tiles && lane == 0 && !(a.agg_only && qs > 0))
        publish(row_status + qs * kSosStatusWords, Alg::affine(G, yin, pv), tag);
      if (lane == 0) s_in = yin;
      __syncthreads();  // entry state is in s_in
      if (v + 2 < nvis)
        build_powers<E, K, R, kWm>(&s_pow[(v + 2) % 3], load_sec(a, b, vis_sec(v + 2)), lane, s_wmat[(v + 2) % 3]);
    }
    return;
  }

  // ================= data waves
  const int pw = REV ? W - 1 - w : w;
  const int pl = REV ? 63 - lane : lane;
  const int64_t seg0 = qf * Sh::kTile + int64_t(pw) * Sh::kWaveSeg;
  auto chunk0 = [&](int r) -> int64_t {  // r in scan order
    const int pr = REV ? R - 1 - r : r;
    return seg0 + int64_t(pr) * 64 * K + int64_t(pl) * K;
  };
  const E zero = E(0);
  int64_t t0s[R];
#pragma unroll
  for (int r = 0; r < R; ++r) t0s[r] = chunk0(r);

  E U[R][K];  // forward: input of the current section;  backward: its upstream gradient
#pragma unroll
  for (int r = 0; r < R; ++r) load_chunk<E, K>(a.in + b * T, chunk0(r), T, vec, U[r], zero);
  // forward values of the current section (x is read again from memory
  // where a re-derivation starts from it, not held in registers)
  E F[GRAD ? R : 1][GRAD ? K : 1];
  if constexpr (GRAD) {
#pragma unroll
    for (int r = 0; r < R; ++r) load_chunk<E, K>(a.x + b * T, chunk0(r), T, vec, F[r], zero);
  }
  if constexpr (ONE) {  // x into the output's slot, for the visit
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int k = 0; k < K; ++k) s_uin[((w * R + r) * K + k) * 64 + lane] = F[r][k];
  }
  __syncthreads();  // powers of the first two visits

  // ---- backward with coefficient gradients: recompute the forward cascade
  // over the lane's chunk from x and the forward's checkpoint of each
  // section's entry state there (the chunk is one checkpoint interval), no
  // scan and no barrier; every lane's entry state of every section stays in
  // LDS for the re-derivations
  if constexpr (GRAD) {
    static_assert(R == 1 && K == kSosCkptEvery<E>, "a lane chunk is one checkpoint interval");
    const int ks = a.kept_step;
    for (int s = 0; s < S; ++s) {
      if (ks > 0 && s > 0 && s % ks == 0 && s / ks <= kSosKeptSlots) {
        E *dst = s_uin + size_t(s / ks - 1) * W * R * K * 64;
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int k = 0; k < K; ++k) dst[((w * R + r) * K + k) * 64 + lane] = F[r][k];
      }
      const SosSec<E> q = load_sec(a, b, s);
      const Vec2<C> *ck = a.ckpt + (b * S + s) * a.n_ckpt;
      SV h[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        h[r] = t0s[r] < T ? Alg::store_s(ck[t0s[r] / kSosCkptEvery<E>]) : SV{zero, zero};
        s_laneh[((s * W + w) * R + r) * 64 + lane] = h[r];
      }
      run_fwd_n<E, K, R>(q, h, F, t0s, T, nullptr);
    }
    // F now holds the cascade output: the forward output of section S-1
  }

  for (int v = 0; v < nvis; ++v) {
    const int s = vis_sec(v);
    const SosSec<E> q = load_sec(a, b, s);
    const SecPowers<C> &t = s_pow[v % 3];
    const SV gzf = load_pair(a.virt + (b * S + s) * 2, REV && a.virt != nullptr);

    E Uf[GRAD ? R : 1][GRAD ? K : 1];

    // ---- pass 1: lane folds, wave scan, round chaining
    V ex[R], tot[R], x[R];
    if constexpr (REV)
      fold_adj_n<E, K, R>(q, U, t0s, T, gzf, x);
    else
      fold_fwd_n<E, K, R>(q, U, x);
    lti_scan<true, REV>(x, lane, t);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      tot[r] = read_lane(x[r], 63);
      ex[r] = lane_prev<true>(x[r], lane, Alg::szero());
    }
    V agg = tot[0];
#pragma unroll
    for (int r = 1; r < R; ++r) agg = mva<REV>(t.pw[64], agg, tot[r]);
    if (lane == 0) s_wagg[w] = M{maybe_transpose<REV>(t.seg), agg};
    __syncthreads();  // wave aggregates are in s_wagg
    // forward input of section s, recomputed from x or from the kept
    // section's input through the sections between (F keeps its output, the
    // previous visit's input), while the look-back wave resolves the entry
    // state (the adjoint's pass 1 does not read it)
    if constexpr (GRAD) {
      const int ks = a.kept_step;
      const int slot = ks > 0 ? (s / ks < kSosKeptSlots ? s / ks : kSosKeptSlots) : 0;  // kept sections <= s
      const int j0 = slot * ks;
      if (ONE || j0 > 0) {
        const E *src = s_uin + size_t(ONE ? 0 : slot - 1) * W * R * K * 64;
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int k = 0; k < K; ++k) Uf[r][k] = src[((w * R + r) * K + k) * 64 + lane];
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r) load_chunk<E, K>(a.x + b * T, chunk0(r), T, vec, Uf[r], zero);
      }
      for (int j = j0; j < s; ++j) {
        const SosSec<E> qj = load_sec(a, b, j);
        SV hj[R];
#pragma unroll
        for (int r = 0; r < R; ++r) hj[r] = s_laneh[((j * W + w) * R + r) * 64 + lane];
        run_fwd_n<E, K, R>(qj, hj, Uf, t0s, T, nullptr);
      }
    }
    __syncthreads();  // entry state is in s_in
    V H = apply<Alg>(s_wpre[w], s_in);

    // ---- pass 2: entry states of every round, then all rounds' steps at once
    SV h[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const V hc = mva<REV>(t.pw[lane], H, ex[r]);
      h[r] = Alg::store_s(hc);
      if constexpr (!REV) {
        if (a.ckpt && (t0s[r] % kSosCkptEvery<E>) == 0 && t0s[r] < T)
          a.ckpt[(b * S + s) * a.n_ckpt + t0s[r] / kSosCkptEvery<E>] = hc;
      }
      H = mva<REV>(t.pw[64], H, tot[r]);
    }
    SosAcc<C> wacc{};
    if constexpr (REV) {
      SosAcc<E> acc[R];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = SosAcc<E>{};
      run_adj_n<E, K, R, GRAD>(q, h, U, t0s, T, gzf, a.fin ? a.fin + (b * S + s) * 2 : nullptr, Uf, F, acc);
      if constexpr (GRAD) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          wacc.a1 += up(acc[r].a1);
          wacc.a2 += up(acc[r].a2);
          wacc.c0 += up(acc[r].c0);
          wacc.c1 += up(acc[r].c1);
          wacc.b0 += up(acc[r].b0);
        }
      }
    } else {
      run_fwd_n<E, K, R>(q, h, U, t0s, T, a.fin ? a.fin + (b * S + s) * 2 : nullptr);
    }
    if constexpr (GRAD) {
      auto sum = [](const SosAcc<C> &p, const SosAcc<C> &o) -> SosAcc<C> {
        return {p.a1 + o.a1, p.a2 + o.a2, p.c0 + o.c0, p.c1 + o.c1, p.b0 + o.b0};
      };
      wacc = wave_scan_incl(wacc, lane, sum);
      if (lane == 63) {
        C *dst = a.partials + ((((b * S + s) * tiles + qf) * W) + w) * 5;
        dst[0] = wacc.a1;
        dst[1] = wacc.a2;
        dst[2] = wacc.c0;
        dst[3] = wacc.c1;
        dst[4] = wacc.b0;
      }
      // the next (lower) section's forward output is this section's input
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int k = 0; k < K; ++k) F[r][k] = Uf[r][k];
    }
  }

  if (a.out) {
    uint4 *wb = nullptr;
    if constexpr (kOutLds) {
      if constexpr (GRAD)
        wb = a.out_lds ? reinterpret_cast<uint4 *>(s_uin + size_t(w) * R * K * 64) : nullptr;
      else
        wb = s_out + w * 64 * kNVo;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t blk0 = chunk0(r) - int64_t(pl) * K;  // the round's block, lowest time first
      if (kOutLds && wb != nullptr && vec && blk0 + 64 * K <= T) {
        if constexpr (kOutLds) {
          lds_put_chunk<E, K>(wb, pl, U[r]);
          lds_flush<kNVo>(reinterpret_cast<uint4 *>(a.out + b * T + blk0), wb, lane, true);
        }
      } else {
        store_chunk<E, K>(a.out + b * T, chunk0(r), T, vec, U[r]);
      }
    }
  }
}

// ------------------------------------------------------------ coefficient gradient
// One block per (coefficient row, section): sums the per-tile, per-wave
// partials (over every batch row when the coefficients are shared) in a fixed
// order and applies the chain rule to (b0, b1, b2, a0, a1, a2):
//   d c0/d b1 = 1, d c0/d b0 = -a1, d c0/d a1 = -b0, d A00/d a1 = -1 (same
//   pattern for c1, a2), d y/d b0 = u; a0 is not a free parameter (zero).
// gsos: [coef_rows, S, 6]; for a biquad given as b and a (a.fb), the
// gradients of whole coefficient tables instead (gsos unused): gb
// [coef_rows, b_cols, nb] with the biquad's b at column b_col and zeros in
// the others, ga [coef_rows, a_cols, 2] likewise (b_cols = a_cols = 1,
// column 0: plain [coef_rows, nb] and [coef_rows, 2]).
constexpr int kSosReduceThreads = 256;

template <typename E, class Sh>
__global__ __launch_bounds__(kSosReduceThreads) void sos_grad_reduce_kernel(const SosArgs<E> a, E *gsos,
                                                                         int64_t coef_rows, E *gb, E *ga,
                                                                         int b_cols, int b_col, int a_cols,
                                                                         int a_col) {
  using C = typename Wide<E>::type;
  __shared__ C s_sum[5][kSosReduceThreads];
  __shared__ C s_g[6];
  const int64_t row = blockIdx.x / a.S;
  const int s = int(blockIdx.x - row * a.S);
  const int64_t per_b = a.tiles_per_row * Sh::kWaves;
  const int64_t b_lo = coef_rows == 1 ? 0 : row, b_hi = coef_rows == 1 ? a.B : row + 1;
  C acc[5] = {C(0), C(0), C(0), C(0), C(0)};
  for (int64_t bb = b_lo; bb < b_hi; ++bb) {
    const C *p = a.partials + ((bb * a.S + s) * per_b) * 5;
    for (int64_t j = threadIdx.x; j < per_b; j += kSosReduceThreads)
#pragma unroll
      for (int c = 0; c < 5; ++c) acc[c] += p[j * 5 + c];
  }
#pragma unroll
  for (int c = 0; c < 5; ++c) s_sum[c][threadIdx.x] = acc[c];
  __syncthreads();
  for (int h = kSosReduceThreads / 2; h > 0; h >>= 1) {
    if (int(threadIdx.x) < h)
#pragma unroll
      for (int c = 0; c < 5; ++c) s_sum[c][threadIdx.x] += s_sum[c][threadIdx.x + h];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const SosCoef<E> k = sec_coef(a, row, s);
    const C b0 = up(k.b0), a1 = up(k.a1), a2 = up(k.a2);
    const C Sa1 = s_sum[0][0], Sa2 = s_sum[1][0], Sc0 = s_sum[2][0], Sc1 = s_sum[3][0], Sb0 = s_sum[4][0];
    const C g[6] = {Sb0 - a1 * Sc0 - a2 * Sc1, Sc0, Sc1, C(0), -Sa1 - b0 * Sc0, -Sa2 - b0 * Sc1};
    if (a.fb) {
#pragma unroll
      for (int j = 0; j < 6; ++j) s_g[j] = g[j];
    } else {
      E *o = gsos + row * int64_t(a.S) * 6 + 6 * s;
#pragma unroll
      for (int j = 0; j < 6; ++j) o[j] = down<E>(g[j]);
    }
  }
  if (a.fb) {
    // the row's tables: the biquad's column, zeros elsewhere
    __syncthreads();
    const int nb = a.nb;
    E *gbr = gb + row * int64_t(b_cols) * nb;
    for (int i = threadIdx.x; i < b_cols * nb; i += kSosReduceThreads) {
      const int col = i / nb;
      gbr[i] = col == b_col ? down<E>(s_g[i - col * nb]) : E(0);
    }
    E *gar = ga + row * int64_t(a_cols) * 2;
    for (int i = threadIdx.x; i < a_cols * 2; i += kSosReduceThreads) {
      const int col = i >> 1;
      gar[i] = col == a_col ? down<E>(s_g[4 + (i & 1)]) : E(0);
    }
  }
}

}  // namespace phs
