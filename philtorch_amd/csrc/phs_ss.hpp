// Fused single-input, single-output LTI state space of order M <= 4 in one
// pass (philtorch/lti/ssm.py:386-589: state_space with a 2D input, B an
// M-vector or absent, C an M-vector or out_idx, D one value per row or absent;
// the glue of lti/ssm.py:467-471, 493-506 and _ssm_C_D :513-589 folded into
// the scan):
//     h[0] = zi,  y[t] = c . h[t] + d x[t],  h[t+1] = A h[t] + b x[t],  zf = h[T]
// Per step one input and one output sample move (the reference route writes
// and reads B x, the state sequence, its shifted copy and C h: about ten
// times the bytes).  Every order runs philtorch's lfilter (companion form,
// TDF-II or DF-II) and state_space for such models.
//
// The decomposition and the look-back are the generic scan's (phs_scan.hpp):
// a lane folds its K steps of (A, b x[t]) from a zero state, wave scans
// chain the lanes, a look-back wave resolves the tile's entry state over the
// row's status words (tagged maps, the generic protocol), and pass 2 re-runs
// the steps from each lane's entry state, writing c . h + d x instead of h.
// Every map's matrix part is a power of A known in advance, so the data
// waves scan vectors only against a table of A^(K 2^i) in LDS (the look-back
// wave builds it while they load): M^2 work and registers per level instead
// of the M^3 of composing maps.  The gradients with respect to x and zi are
// this kernel on the adjoint model (A^T, input vector c, output vector b, d,
// run in the opposite time direction from dL/dzf).  Those of the
// coefficients take two launches (ss_grad_* below): a forward that writes
// the state before every step (kSsStates), then the adjoint pass
// (kSsGrad), which at every step also has the adjoint state lambda[t+1]
// = dL/dh[t+1], the upstream gradient g[t], the forward state h[t] and the
// input x[t] in hand and sums, per wave,
//     dL/dA = sum_t lambda[t+1] h[t]^T,  dL/db = sum_t lambda[t+1] x[t],
//     dL/dc = sum_t g[t] h[t],           dL/dd = sum_t g[t] x[t],
// the gradient of the composed graph the reference differentiates
// (philtorch/lti/ssm.py:467-589, filtering.py:273-333).
//
// The same kernel runs both passes of a zero-phase filter (philtorch/lti/
// filtering.py:413-484 filtfilt): scan positions map to descending time
// (REV), and a row's entry state is derived in the kernel from the edge of
// the row (ss_filtfilt_entry), so that neither the padded copy nor the flips
// exist.
#pragma once

#include "phs_scan.hpp"

namespace phs {

template <class Alg>
struct SsArgs {
  using E = typename Alg::elem;
  const E *A;         // [rows, M, M] row-major
  int64_t A_stride;   // elements between rows (0 = shared)
  int A_trans;        // use A^T (the adjoint model of an explicit A)
  const E *bv;        // [rows, M]; nullptr: the input enters state in_idx
  int64_t b_stride;
  int in_idx;
  const E *cv;        // [rows, M]; nullptr: y is state out_idx
  int64_t c_stride;
  const E *d;         // [rows]; nullptr: no feedthrough
  int64_t d_stride;
  int out_idx;
  // filter mode (filt_form != 0: A, bv, cv, d are not read): the model of
  // lfilter(fb, fa) in companion form, fb [rows, nb] (nb <= M + 1) and fa
  // [rows, na] (the denominator after its leading 1, na <= M), both
  // zero-padded to order M (philtorch/lti/filtering.py:273-333):
  //   1 TDF-II: A = companion(a)^T, b = fb[1:] - fb[0] a, c = e0, d = fb[0]
  //   2 DF-II:  A = companion(a),   b = e0, c = fb[1:] - fb[0] a, d = fb[0]
  const E *fb, *fa;
  int nb, na, filt_form;
  int64_t f_stride_b, f_stride_a;  // 0 = shared
  const E *zi;        // [B, M]; nullptr: zeros
  // The rows' entry states (virt_mode): 0 zi above; 1 and 2 the two passes
  // of a zero-phase filter (ss_filtfilt_entry below): 1 the steady state of
  // the padded row's first sample, stepped over the front pad of xpad; 2 the
  // state pass 1 (final state zf_prev) reaches over the back pad, carried
  // into the time-reversed pass
  int virt_mode;
  const E *xpad;      // [B, T] the zero-phase filter's input (pad values)
  const E *zf_prev;   // [B, M] pass 1's final state (virt_mode 2)
  int pad_mode;
  int64_t pad_len;
  const E *x;         // [B, T]
  E *y;               // [B, T]
  E *zf;              // [B, M]; nullable (scan order: the state after the last step scanned)
  // kSsStates: the state before every step, [B, T, M] at its time index
  // (y is not written); kSsGrad: the forward's states and input, read at
  // every step, and the per-wave coefficient-gradient sums
  // [B, tiles_per_row, kWaves, SsGradN] in compute precision
  E *hs;
  const E *hs_fwd, *x_fwd;
  typename Wide<E>::type *gpart;
  int vec_hs;         // 16-byte state chunks (T M sizeof(E) % 16 == 0, aligned)
  int64_t B, T_len, tiles_per_row;
  unsigned long long *claims;
  unsigned tiles, per_stripe, spin_limit;
  unsigned agg_only;  // testing: tiles after a row's first publish no inclusive state
  uint64_t b_magic;   // tile id -> row by multiply and shift (row_split)
  unsigned b_shift;
  uint64_t *status;
  int vec_ok;
  // plain forward of a second-order model (nullable): the state entering
  // every ckpt_every-th step, in compute precision, [B, n_ckpt] (the
  // checkpoints the fused cascade's gradient backward reads at one section)
  void *ckpt;
  int64_t n_ckpt;
  int ckpt_every;
};

// Kernel modes: the model's output (plain), the states of a forward for the
// coefficient gradients (kSsStates: h[t] before every step, no y), the
// adjoint pass with the coefficient-gradient sums (kSsGrad), the states
// and the output with the final state (kSsStatesY: a zero-phase filter's
// first pass, whose output is the second pass's input).
constexpr int kSsPlain = 0, kSsStates = 1, kSsGrad = 2, kSsStatesY = 3;

// 3 data waves and a look-back wave.  Orders 1-2: 4 rounds of two 16-byte
// vectors of inputs per lane (8 fp32 or 4 fp64 steps); orders 3-4: 2 rounds
// of four vectors, which halves the scan levels per step where each level
// is an M x M product (6144-step fp32 tiles either way; at the C4 shape,
// order 4 takes 53 us per launch against 67 with the other split and 74
// with 3072-step tiles, order 1 25 against 28).  The gradient mode runs
// half the rounds (3072-step fp32 tiles): its sums and the forward's states
// take the registers the other rounds' inputs would, and the order-4
// adjoint spilled.  At the C4 shape a backward call with coefficient
// gradients (states pass, adjoint, sums) went 279 -> 237 us at order 4,
// 217 -> 188 at order 3, 134 -> 128.5 at order 2 and 86.5 -> 85.5 at
// order 1; the other modes are slower with fewer rounds.
//
// The fp32 order-2 plain pass is a wide tile instead: 15 data waves of 16
// steps in 2 rounds (30720 steps) beside the look-back wave, held to 128
// VGPRs (four waves per SIMD; 98 used), so one tile fills a CU's wave
// slots and a C4 call is 256 tiles all resident at once, where 3-wave tiles
// at 158 VGPRs were 1264 tiles on 768 resident slots (two generations).
template <class Alg, int MODE = kSsPlain>
struct SsShape {
  using E = typename Alg::elem;
  static constexpr int M = int(sizeof(typename Alg::s_state) / sizeof(E));
  static constexpr bool kWide = MODE == kSsPlain && M == 2 && sizeof(E) == 4;
  static constexpr int kWaves = kWide ? 15 : 3;
  static constexpr int kMinWaves = kWide ? 4 : 2;  // waves per SIMD the launch bounds ask for
  static constexpr int kThreads = 64 * (kWaves + 1);
  static constexpr int K = kWide ? 16 : int((M <= 2 ? 32 : 64) / sizeof(E));
  static constexpr int R = kWide ? 2 : (M <= 2 ? 4 : 2) / (MODE == kSsGrad ? 2 : 1);
  static constexpr int kWaveSeg = 64 * K * R;
  static constexpr int kTile = kWaves * kWaveSeg;
  // The last kLdsRounds rounds' inputs wait in LDS between the passes.  The
  // wide tile's second round (61 KB of the CU's 160) took it from 128 VGPRs
  // with 32 (reversed 48) bytes a lane spilled to scratch, whose traffic
  // reached HBM, to 98 (92) and none: 26.5 -> 25.7 us forward at the C4
  // shape, reversed unchanged.  Both rounds measured no faster.
  static constexpr int kLdsRounds = kWide ? 1 : 0;
  static_assert((K & (K - 1)) == 0, "K is a power of two (the lane matrix is A^K by squaring)");
};

// Chunk I/O in scan order: forward, scan position s is time s; reversed
// (REV), it is time T-1-s, so a lane's K steps are the K samples below
// T - s0, read (and written) in descending time.  Positions past the row
// read 0 and are not written.  The bounds-checked paths assign in branches
// (no select between a global and a private address).  kFull: the chunk
// is known to be in range and aligned, only the vector form is compiled.
template <bool REV, typename E, int K, bool kFull = false>
__device__ __forceinline__ void ss_load(const E *row, int64_t s0, int64_t T, bool vec, E (&out)[K]) {
  if constexpr (!REV) {
    load_chunk<E, K, kFull>(row, s0, T, vec, out, E{});
  } else {
    const int64_t base = T - s0 - K;  // lowest time of the chunk
    if (kFull || (vec && base >= 0)) {
      E tmp[K];
      load_chunk<E, K>(row, base, T, true, tmp, E{});
#pragma unroll
      for (int k = 0; k < K; ++k) out[k] = tmp[K - 1 - k];
    } else {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int64_t t = T - 1 - s0 - k;
        if (t >= 0)
          out[k] = row[t];
        else
          out[k] = E{};
      }
    }
  }
}

template <bool REV, typename E, int K, bool kFull = false>
__device__ __forceinline__ void ss_store(E *row, int64_t s0, int64_t T, bool vec, const E (&v)[K]) {
  static_assert(K * sizeof(E) % 16 == 0, "whole 16-byte vectors");
  if constexpr (!REV) {
    store_chunk<E, K, kFull>(row, s0, T, vec, v);
  } else {
    const int64_t base = T - s0 - K;
    if (kFull || (vec && base >= 0)) {
      E tmp[K];
#pragma unroll
      for (int k = 0; k < K; ++k) tmp[k] = v[K - 1 - k];
      store_chunk<E, K>(row, base, T, true, tmp);
    } else {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int64_t t = T - 1 - s0 - k;
        if (t >= 0) row[t] = v[k];
      }
    }
  }
}

// padmode codes (PHS_PAD_* in philscan.h): torch.nn.functional.pad modes
constexpr int kPadConstant = 0;   // zeros
constexpr int kPadReplicate = 1;  // edge value
constexpr int kPadReflect = 2;    // mirror without repeating the edge
constexpr int kPadCircular = 3;   // wrap around

// ext[j] for j in [0, e): the front pad of a row of T samples (e < T)
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

// The element view of a state or coefficient (Scalar: one value, Block2 and
// BlockN: contiguous fields in index order).
template <class Alg>
struct SsView {
  using E = typename Alg::elem;
  using SS = typename Alg::s_state;
  using SC = typename Alg::s_coef;
  static constexpr int M = int(sizeof(SS) / sizeof(E));
  static_assert(sizeof(SC) == sizeof(E) * M * M, "row-major M x M coefficient");

  static __device__ __forceinline__ SS load_vec(const E *p) {
    union {
      SS s;
      E e[M];
    } u;
#pragma unroll
    for (int i = 0; i < M; ++i) u.e[i] = p[i];
    return u.s;
  }
  static __device__ __forceinline__ SS unit(int i) {
    union {
      SS s;
      E e[M];
    } u;
#pragma unroll
    for (int j = 0; j < M; ++j) u.e[j] = j == i ? E(1) : E(0);
    return u.s;
  }
  static __device__ __forceinline__ SC load_mat(const E *p) {
    union {
      SC s;
      E e[M * M];
    } u;
#pragma unroll
    for (int i = 0; i < M * M; ++i) u.e[i] = p[i];
    return u.s;
  }
  // b x
  static __device__ __forceinline__ SS scale(const SS &b, E x) {
    union {
      SS s;
      E e[M];
    } u, o;
    u.s = b;
#pragma unroll
    for (int i = 0; i < M; ++i) o.e[i] = u.e[i] * x;
    return o.s;
  }
  // c . h
  static __device__ __forceinline__ E dot(const SS &c, const SS &h) {
    union {
      SS s;
      E e[M];
    } uc, uh;
    uc.s = c;
    uh.s = h;
    E acc = uc.e[0] * uh.e[0];
#pragma unroll
    for (int i = 1; i < M; ++i) acc = fma(uc.e[i], uh.e[i], acc);
    return acc;
  }
};

// The model of row b in storage precision (a shared operand has stride 0).
template <class Alg>
struct SsModel {
  using E = typename Alg::elem;
  typename Alg::s_coef A;
  typename Alg::s_state b, c;
  E d;
};

// kAdjoint: honour A_trans and in_idx (set only for the adjoint pass of the
// coefficient gradients; the other modes read A as it lies, input state 0).
template <class Alg, bool kAdjoint = false>
__device__ __forceinline__ SsModel<Alg> ss_model(const SsArgs<Alg> &a, int64_t row) {
  using V = SsView<Alg>;
  using E = typename Alg::elem;
  constexpr int M = V::M;
  SsModel<Alg> m;
  // Every coefficient is read before any is used, with no branch around a
  // read (absent operands read an in-bounds stand-in and are selected away
  // after), so the reads overlap in one round trip instead of one each.
  if (a.filt_form == 0) {
    const E *pA = a.A + row * a.A_stride;
    const E *pb = a.bv ? a.bv + row * a.b_stride : pA;
    const E *pc = a.cv ? a.cv + row * a.c_stride : pA;
    const E *pd = a.d ? a.d + row * a.d_stride : pA;
    const typename Alg::s_coef Am = V::load_mat(pA);
    const typename Alg::s_state bl = V::load_vec(pb), cl = V::load_vec(pc);
    const E dl = pd[0];
    m.A = Am;
    if (kAdjoint && a.A_trans) m.A = Alg::s_adjoint(m.A);  // real: the transpose
    m.b = a.bv ? bl : V::unit(kAdjoint ? a.in_idx : 0);
    m.c = a.cv ? cl : V::unit(a.out_idx);
    m.d = a.d ? dl : E(0);
    return m;
  }
  const E *fb = a.fb + row * a.f_stride_b, *fa = a.fa + row * a.f_stride_a;
  E fav[M], fbv[M + 1];  // nb >= 1 and na >= 1: index 0 is always in range
#pragma unroll
  for (int i = 0; i < M; ++i) fav[i] = fa[i < a.na ? i : 0];
#pragma unroll
  for (int i = 0; i <= M; ++i) fbv[i] = fb[i < a.nb ? i : 0];
#pragma unroll
  for (int i = 0; i < M; ++i) fav[i] = i < a.na ? fav[i] : E(0);
#pragma unroll
  for (int i = 0; i <= M; ++i) fbv[i] = i < a.nb ? fbv[i] : E(0);
  union {
    typename Alg::s_coef s;
    E e[M * M];
  } A;
  union {
    typename Alg::s_state s;
    E e[M];
  } g;
  const E b0 = fbv[0];
#pragma unroll
  for (int i = 0; i < M; ++i) {
    g.e[i] = fbv[i + 1] - b0 * fav[i];
#pragma unroll
    for (int j = 0; j < M; ++j) {
      // companion(a): row 0 = -a, ones below the diagonal
      const E comp_ij = i == 0 ? -fav[j] : (j == i - 1 ? E(1) : E(0));
      const E comp_ji = j == 0 ? -fav[i] : (i == j - 1 ? E(1) : E(0));
      A.e[i * M + j] = a.filt_form == 1 ? comp_ji : comp_ij;
    }
  }
  m.A = A.s;
  m.b = a.filt_form == 1 ? g.s : V::unit(0);
  m.c = a.filt_form == 1 ? V::unit(0) : g.s;
  m.d = b0;
  return m;
}

// The TDF-II model of lfilter(fb, fa) of order M in double (filter form 1:
// h' = A h + g u with A = companion(a)^T, g = b[1:] - b0 a, y = h0 + b0 u)
// and its steady state for a unit input z = (I - A)^-1 g (lfilter_zi,
// philtorch/lti/filtering.py:107-142), from the companion structure:
// z0 = H(1) - b0 with H(1) = sum(b) / (1 + sum(a)), z(i+1) = z(i) + a_i z0
// - g_i.
template <int M>
struct FfModel {
  double am[M], g[M], z[M], b0;
};
template <int M, typename E>
__device__ __forceinline__ FfModel<M> ff_model(const E *fb, int nb, const E *fa, int na) {
  FfModel<M> f;
  f.b0 = double(fb[0]);
  double sb = f.b0, sa = 1.0;
#pragma unroll
  for (int i = 0; i < M; ++i) {
    f.am[i] = i < na ? double(fa[i]) : 0.0;
    const double bi = i + 1 < nb ? double(fb[i + 1]) : 0.0;
    f.g[i] = bi - f.b0 * f.am[i];
    sb += bi;
    sa += f.am[i];
  }
  f.z[0] = sb / sa - f.b0;
#pragma unroll
  for (int i = 0; i + 1 < M; ++i) f.z[i + 1] = f.z[i] + f.am[i] * f.z[0] - f.g[i];
  return f;
}

// Entry state of row b for the two passes of a zero-phase filter
// (virt_mode 1 and 2), in double, on the TDF-II model of lfilter(fb, fa) of
// order M (filter form 1: h' = A h + g u with A = companion(a)^T, g = b[1:]
// - b0 a, y = h0 + b0 u).  Both passes run that one model whatever form the
// caller names: each starts from the steady state of the same transfer
// function, so the outputs are the same (the reference runs its `form`).
//
//  * z the steady state of a unit input (ff_model);
//  * pass 1 starts at z ext[0] before the e front-pad samples of xpad, so
//    its entry state is that stepped over them (filtering.py:466-470);
//  * pass 2 filters the reversed pass-1 output over the padded row, whose
//    first e samples are the back pad's outputs yb[e-1..0] (pass 1 stepped
//    on from its final state zf_prev over the back pad of xpad), from
//    z yb[e-1] (z y1[T-1] if e = 0; filtering.py:472-474).  Folded:
//        h = A^e z y0 + sum_j A^j g yb[j].
// A filter with a pole at z = 1 (1 + sum(a) = 0) has no steady state: the
// reference's linalg.solve raises, here the output is not finite.
// Tile 0 of a row derives it while its data loads (and the look-back's
// fallback), every lane the same: the pad samples are loaded 64 at a time,
// one per lane, so the serial steps wait on one load latency per batch
// rather than one per sample.
template <class Alg>
__device__ __forceinline__ typename Alg::state ss_filtfilt_entry(const SsArgs<Alg> &a, int64_t b, int lane) {
  using E = typename Alg::elem;
  constexpr int M = SsView<Alg>::M;
  const FfModel<M> f = ff_model<M>(a.fb + b * a.f_stride_b, a.nb, a.fa + b * a.f_stride_a, a.na);
  const double b0 = f.b0;
  const double(&am)[M] = f.am;
  const double(&g)[M] = f.g;
  const double(&z)[M] = f.z;
  double h[M];
  // h <- A h + g u (ascending i reads h[i+1] before it changes)
  auto step = [&](double (&v)[M], double u) {
    const double v0 = v[0];
#pragma unroll
    for (int i = 0; i < M; ++i) v[i] = -am[i] * v0 + (i + 1 < M ? v[i + 1] : 0.0) + g[i] * u;
  };
  const int64_t T = a.T_len, e = a.pad_len;
  const E *xp = a.xpad + b * T;
  if (a.virt_mode == 1) {
    const double u0 = double(e > 0 ? pad_front(xp, T, e, a.pad_mode, 0) : xp[0]);
#pragma unroll
    for (int i = 0; i < M; ++i) h[i] = z[i] * u0;
    for (int64_t j0 = 0; j0 < e; j0 += 64) {
      const int64_t jl = j0 + lane;
      const double ul = jl < e ? double(pad_front(xp, T, e, a.pad_mode, jl)) : 0.0;
      const int n = e - j0 < 64 ? int(e - j0) : 64;
      for (int j = 0; j < n; ++j) step(h, read_lane(ul, j));
    }
  } else {
    double P[M][M], acc[M], ul = 0.0;
#pragma unroll
    for (int i = 0; i < M; ++i) {
      h[i] = double(a.zf_prev[b * M + i]);
      acc[i] = 0.0;
#pragma unroll
      for (int k = 0; k < M; ++k) P[i][k] = i == k ? 1.0 : 0.0;
    }
    double y0 = e > 0 ? 0.0 : double(a.x[b * T + T - 1]);
    for (int64_t j = 0; j < e; ++j) {
      if ((j & 63) == 0) {  // the next batch of back-pad samples, one per lane
        const int64_t jl = j + lane;
        ul = jl < e ? double(pad_back(xp, T, a.pad_mode, jl)) : 0.0;
      }
      const double u = read_lane(ul, int(j & 63));
      const double yb = h[0] + b0 * u;
      // acc += A^j g yb, then P = A^(j+1) (row i: -a_i P[0] + P[i+1])
#pragma unroll
      for (int i = 0; i < M; ++i) {
        double t = 0.0;
#pragma unroll
        for (int k = 0; k < M; ++k) t += P[i][k] * g[k];
        acc[i] += t * yb;
      }
      double p0[M];
#pragma unroll
      for (int k = 0; k < M; ++k) p0[k] = P[0][k];
#pragma unroll
      for (int i = 0; i < M; ++i)
#pragma unroll
        for (int k = 0; k < M; ++k) P[i][k] = -am[i] * p0[k] + (i + 1 < M ? P[i + 1][k] : 0.0);
      step(h, u);
      y0 = yb;
    }
#pragma unroll
    for (int i = 0; i < M; ++i) {
      double t = acc[i];
#pragma unroll
      for (int k = 0; k < M; ++k) t += P[i][k] * z[k] * y0;
      h[i] = t;
    }
  }
  union {
    typename Alg::s_state s;
    E e[M];
  } u;
#pragma unroll
  for (int i = 0; i < M; ++i) u.e[i] = E(h[i]);
  return Alg::load_s(u.s);
}

// A^(2^n) in compute precision.
template <class Alg>
__device__ __forceinline__ typename Alg::coef ss_pow2(const typename Alg::s_coef &A, int n) {
  typename Alg::coef P = Alg::load_c(A);
  for (int i = 0; i < n; ++i) P = Alg::cmul(P, P);
  return P;
}

// A lane's K steps from a zero state, sum_k A^(K-1-k) b x[k] (the vector
// part of its map; the matrix part is A^K).
template <class Alg, int K>
__device__ __forceinline__ typename Alg::state ss_lane_fold(const SsModel<Alg> &m,
                                                            const typename Alg::elem (&x)[K]) {
  using V = SsView<Alg>;
  typename Alg::s_state h = V::scale(m.b, x[0]);
#pragma unroll
  for (int k = 1; k < K; ++k) h = Alg::s_affine(m.A, h, V::scale(m.b, x[k]));
  return Alg::load_s(h);
}

// Status entries carry vectors only: every tile aggregate has the matrix
// part G = A^(tile steps), so an entry is the inclusive state (words
// [0, kVecWords)) and the tile's zero-entry aggregate (the next kVecWords),
// each 32-bit chunk one tagged 64-bit word as in phs_scan.hpp.
template <class Alg>
struct SsStatus {
  static constexpr int kVecWords = int(sizeof(typename Alg::state) / 4);
  static constexpr int kStride = 2 * kVecWords;
  static constexpr int kLookPitch = kStride | 1;  // odd LDS pitch: no bank conflicts
  static constexpr int kLookWords = 64 * kLookPitch;
};

// Power tables the look-back wave builds in LDS before the data waves scan:
// pw[i] = A^(K 2^i) (i < 6) for the lane scan, pw[6] = A^(64 K) between
// rounds, pw[7] = A^(64 K R) per wave segment; gp[j] = G^(2^j) (j < 7) for
// the look-back, G = A^(tile steps).
template <class Alg>
struct SsPowers {
  typename Alg::coef pw[8];
  typename Alg::coef gp[7];
};

// The power tables live in LDS and are read where they are used: a compiler
// barrier at the top of each loop keeps their loads from being hoisted out
// of it, where up to six M x M matrices would sit in registers at once.
__device__ __forceinline__ void ss_reload_tables() { asm volatile("" ::: "memory"); }

// v[r] <- P^n v[r] for a table P[j] = P^(2^j) and 0 <= n < 2^bits, level by
// level so that one matrix serves every vector (powers of one matrix
// commute, so the order of the factors is free).
template <class Alg, int Bits, int N>
__device__ __forceinline__ void ss_pow_apply(const typename Alg::coef *P, int n, typename Alg::state (&v)[N]) {
#pragma unroll
  for (int j = 0; j < Bits; ++j) {
    if ((n >> j) & 1) {
      const typename Alg::coef Pj = P[j];
#pragma unroll
      for (int r = 0; r < N; ++r) v[r] = Alg::affine(Pj, v[r], Alg::szero());
    }
  }
}

// A lane's place in the scan order.  FLIP (the reversed pass) numbers the
// lanes from 63 down, so that lanes in ascending order still read and write
// ascending addresses when scan positions run down in time; the scans below
// then combine with the lane above rather than below.
template <bool FLIP>
__device__ __forceinline__ int ss_scan_lane(int lane) {
  return FLIP ? 63 - lane : lane;
}
template <bool FLIP>
__device__ __forceinline__ int ss_last_lane() {
  return FLIP ? 0 : 63;
}

// Inclusive scans of N rounds of lane vectors, v_L = sum_{j <= L}
// A^(K (L-j)) s_j over scan lanes L: Kogge-Stone, level i combines with the
// scan lane 2^i below at A^(K 2^i), level by level across the rounds.
template <class Alg, int N, bool FLIP>
__device__ __forceinline__ void ss_lane_scan(typename Alg::state (&v)[N], int lane, const typename Alg::coef *pw) {
  const int sl = ss_scan_lane<FLIP>(lane);
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    const int d = 1 << i;
    typename Alg::state o[N];
#pragma unroll
    for (int r = 0; r < N; ++r) o[r] = shfl_from(v[r], FLIP ? lane + d : lane - d);
    if (sl >= d) {
      const typename Alg::coef P = pw[i];
#pragma unroll
      for (int r = 0; r < N; ++r) v[r] = Alg::affine(P, o[r], v[r]);
    }
  }
}

// State entering scan position `span` of a row, folded straight from the
// inputs (the look-back's bounded-wait fallback; out of line, cold): chunk
// by chunk of 64 K steps, st <- A^(64 K) st + chunk total, from the row's
// entry state st (derived here for a zero-phase pass).
template <class Alg, class Sh, bool REV, bool kAdjoint>
__device__ __noinline__ typename Alg::state ss_prefix_fallback(const SsArgs<Alg> *ap, int64_t b, int64_t span,
                                                              int lane, typename Alg::state st,
                                                              const SsPowers<Alg> *tab) {
  const SsArgs<Alg> &a = *ap;
  using E = typename Alg::elem;
  constexpr int K = Sh::K;
  const SsModel<Alg> m = ss_model<Alg, kAdjoint>(a, b);
  const E *xrow = a.x + b * a.T_len;
  if (a.virt_mode != 0) st = ss_filtfilt_entry<Alg>(a, b, lane);
  for (int64_t off = 0; off < span; off += 64 * K) {
    ss_reload_tables();
    E xs[K];
    ss_load<REV, E, K>(xrow, off + int64_t(ss_scan_lane<REV>(lane)) * K, a.T_len, a.vec_ok != 0, xs);
    typename Alg::state v[1] = {ss_lane_fold<Alg, K>(m, xs)};
    ss_lane_scan<Alg, 1, REV>(v, lane, tab->pw);
    st = Alg::affine(tab->pw[6], st, read_lane(v[0], ss_last_lane<REV>()));
  }
  return st;
}

// One tile's look-back over vector entries: with lane i looking at tile
// q-1-i and k the first lane holding an inclusive state, the state entering
// tile q is sum_{i<k} G^i agg(q-1-i) + G^k inc(q-1-k) (windows further back
// weighted by G^(tiles passed)).  The first window holds Alg::kLookFirst
// tiles, later ones 64.  Polls until the state is known (true, in `out`) or
// `spin_limit` polls found a predecessor still unpublished (false).
template <class Alg>
__device__ bool ss_lookback(const uint64_t *row_status, const typename Alg::state &virt, int lane, unsigned tag,
                            unsigned spin_limit, uint64_t *s_look, const SsPowers<Alg> *tab, int64_t q,
                            typename Alg::state &out) {
  using S = typename Alg::state;
  using Mt = typename Alg::coef;
  using St = SsStatus<Alg>;
  constexpr int kS = St::kStride, kP = St::kLookPitch, kV = St::kVecWords;
  constexpr int kBatch = kS < 8 ? kS : 8;  // words in flight per lane
  S acc = Alg::szero();
  Mt gm = Alg::cone();
  int64_t base = q - 1;
  unsigned polls = 0;
  int span = Alg::kLookFirst;
  auto add = [](const S &p, const S &o) { return Alg::sadd(p, o); };
  while (true) {
    ss_reload_tables();
    const int n = base + 1 > span ? span : int(base + 1);  // tiles in the window
    const uint64_t *win = row_status + (base + 1 - n) * kS + lane;
    // all loads of a batch are issued before any LDS store (atomic loads are
    // ordered against other memory operations)
#pragma unroll
    for (int i0 = 0; i0 < kS; i0 += kBatch) {
      uint64_t words[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        words[i] = 0;
        if (i0 + i < kS && (i0 + i) * 64 + lane < n * kS)  // word (i0+i)*64+lane of the window
          words[i] = __hip_atomic_load(win + (i0 + i) * 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int j = (i0 + i) * 64 + lane;
        if (i0 + i < kS) s_look[(j / kS) * kP + (j % kS)] = words[i];
      }
    }
    wave_sync();
    const int64_t p = base - lane;  // lane < n: window entry n-1-lane
    S inc = Alg::szero(), agg = Alg::szero();
    int st = 3;  // outside the window: no contribution, never inclusive
    if (lane < n) {
      const uint64_t *e = s_look + (n - 1 - lane) * kP;
      const bool inc_ok = unpack(e, inc, tag);
      const bool agg_ok = unpack(e + kV, agg, tag);
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
    S c[1] = {Alg::szero()};
    if (lane < k && lane < n) c[0] = agg;
    if (lane == k) c[0] = inc;
    ss_pow_apply<Alg, 6, 1>(tab->gp, lane, c);
    const S sum = read_lane(wave_scan_incl(c[0], lane, add), 63);
    acc = Alg::affine(gm, sum, acc);
    if (k < 64) {
      out = acc;
      return true;
    }
    // G^n for the window just passed (n = kLookFirst or 64, a power of two)
    gm = Alg::cmul(n == 64 ? tab->gp[6] : tab->gp[__builtin_ctz(unsigned(n))], gm);
    base -= n;
    span = 64;
  }
}

// Coefficient-gradient sums of one model: dL/dA (M x M row-major), dL/db
// (M), dL/dc (M), dL/dd; a lane sums its own steps in storage precision
// (32 fp32 or 16 fp64 steps), everything above it in compute precision.
template <class Alg, typename V = typename Wide<typename Alg::elem>::type>
struct SsGrad {
  static constexpr int M = SsView<Alg>::M;
  static constexpr int kA = 0, kB = M * M, kC = M * M + M, kD = M * M + 2 * M, kN = M * M + 2 * M + 1;
  V v[kN];
};

// Steps per group of state loads and stores: at most 64 bytes of states
// and whole 16-byte vectors of states and inputs (bounds the registers a
// K-step chunk of order-4 states would take).  A 32-byte group in the
// gradient mode removed the order-2 fp32 reversed adjoint's 9 spilled
// registers but measured no faster there and 6% slower forward.
template <class Alg>
constexpr int ss_state_group() {
  constexpr int K = SsShape<Alg>::K;
  constexpr int bytes = int(sizeof(typename Alg::s_state));
  int g = 1;
  while (2 * g <= K && 2 * g * bytes <= 64) g *= 2;
  return g;
}

// One step's contribution: lambda = dL/dh[t+1] (the adjoint state before
// the step), hf = h[t], xf = x[t], g = dL/dy[t].
template <class Alg>
__device__ __forceinline__ void ss_grad_step(SsGrad<Alg, typename Alg::elem> &acc,
                                             const typename Alg::s_state &lambda, const typename Alg::s_state &hf,
                                             typename Alg::elem xf, typename Alg::elem g) {
  using E = typename Alg::elem;
  using G = SsGrad<Alg, E>;
  constexpr int M = G::M;
  union {
    typename Alg::s_state s;
    E e[M];
  } ul, uh;
  ul.s = lambda;
  uh.s = hf;
#pragma unroll
  for (int i = 0; i < M; ++i) {
    const E li = ul.e[i];
#pragma unroll
    for (int j = 0; j < M; ++j) acc.v[G::kA + i * M + j] = fma(li, uh.e[j], acc.v[G::kA + i * M + j]);
    acc.v[G::kB + i] = fma(li, xf, acc.v[G::kB + i]);
    acc.v[G::kC + i] = fma(g, uh.e[i], acc.v[G::kC + i]);
  }
  acc.v[G::kD] = fma(g, xf, acc.v[G::kD]);
}

// At least two waves per SIMD (two workgroups per CU; wide tiles four).
// Group g0 .. g0+G-1 of a lane's K steps (items of type X, whole 16-byte
// vectors) into the wave's lane-blocked buffer `wb` (lds_flush's layout), in
// ascending time (a reversed pass walks its chunk downwards).
template <int NV, bool REV, int K, typename X, int G>
__device__ __forceinline__ void ss_lds_put(uint4 *wb, int lane, int g0, const X (&items)[G]) {
  constexpr int NG = int(G * sizeof(X) / 16);
  static_assert(G * sizeof(X) % 16 == 0 && K % G == 0, "whole vectors");
  union {
    X x[G];
    uint4 u[NG];
  } t;
#pragma unroll
  for (int i = 0; i < G; ++i) t.x[i] = items[REV ? G - 1 - i : i];
  const int v0 = int((REV ? K - g0 - G : g0) * sizeof(X) / 16);
  const int sw = lds_swizzle<NV>(lane);
#pragma unroll
  for (int i = 0; i < NG; ++i) wb[lane * NV + ((v0 + i) ^ sw)] = t.u[i];
}


// A workgroup barrier with no wait for outstanding memory operations, whose
// memory accesses stay on their side of it: memory operations issued before
// it by one wave are queued ahead of those the others issue after it.
__device__ __forceinline__ void issue_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <class Alg, bool REV, int MODE>
__global__ __launch_bounds__((SsShape<Alg, MODE>::kThreads), (SsShape<Alg, MODE>::kMinWaves)) void ss_kernel(
    SsArgs<Alg> a) {
  using E = typename Alg::elem;
  using S = typename Alg::state;
  using SS = typename Alg::s_state;
  using V = SsView<Alg>;
  using Sh = SsShape<Alg, MODE>;
  using St = SsStatus<Alg>;
  constexpr int K = Sh::K, R = Sh::R, kWaves = Sh::kWaves;
  static_assert(Alg::kLookFirst == 8 || Alg::kLookFirst == 64, "window weights are table entries");

  __shared__ S s_wagg[kWaves];  // wave aggregates (matrix part A^(64 K R))
  __shared__ S s_wpre[kWaves];  // exclusive wave prefixes (matrix part A^(64 K R w))
  __shared__ S s_in;
  __shared__ unsigned s_id, s_tag;
  __shared__ uint64_t s_look[St::kLookWords];
  __shared__ SsPowers<Alg> s_tab;
  __shared__ SsModel<Alg> s_model;  // the row's model, from the look-back wave
  // inputs of the rounds that wait in LDS, 16 bytes a lane at a time, lanes
  // adjacent: [wave][round][vector][lane]
  constexpr int kLR = Sh::kLdsRounds;
  constexpr int kEV = int(16 / sizeof(E));  // elements per 16-byte vector
  struct alignas(16) Vec16 {
    E e[kEV];
  };
  __shared__ Vec16 s_xin[kLR > 0 ? kWaves * kLR * (K / kEV) * 64 : 1];
  // Outputs and states of full tiles leave through LDS: a lane's K steps
  // are K consecutive samples, so a 16-byte store instruction of the lanes
  // themselves touches 64 separate segments; transposed, each instruction
  // writes 1 KB of the row in one piece.  [wave][lane-blocked vectors,
  // swizzled], one round at a time.  At the C4 shape (fp32): order-2
  // lfilter 25.7 -> 22.3 us forward and 26.5 -> 22.0 reversed (a plain
  // copy in the wide tile's geometry takes 26.6 us lane-blocked, 21.7
  // transposed), the order-2 states pass 38.2 -> 29.5, order 4's 69.6 ->
  // 57.2, order 1 23.0 -> 22.2.  The plain pass of orders 3-4 (2.5
  // generations of tiles, 4 x 4 steps) ran 49 -> 53 us forward with it and
  // keeps its lanes' stores.
  constexpr bool kStates = MODE == kSsStates || MODE == kSsStatesY;
  constexpr int kNVy = int(K * sizeof(E) / 16);   // 16-byte vectors of outputs per lane and round
  constexpr int kNVh = int(K * sizeof(SS) / 16);  // of states
  constexpr bool kYLds = MODE != kSsStates && !(MODE == kSsPlain && V::M >= 3) && kNVy > 1;
  constexpr bool kHLds = kStates && kNVh > 1 && (kNVh & (kNVh - 1)) == 0 && kNVh <= 16 &&
                         int(K * sizeof(SS)) % 16 == 0;
  __shared__ uint4 s_yt[kYLds ? kWaves * 64 * kNVy : 1];
  __shared__ uint4 s_ht[kHLds ? kWaves * 64 * kNVh : 1];

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
  int64_t q, b;  // tile position along the row, row
  split_tile(id, a.B, a.b_magic, a.b_shift, q, b);
  const int64_t T = a.T_len;

  if (w == kWaves) {
    // ================= look-back wave: power tables, then the look-back
    {
      // the model's reads go out before the data waves' input loads (the
      // barrier below, without a wait, releases them): the power tables,
      // which the data waves wait for, start as soon as the model is in
      const SsModel<Alg> mrow = ss_model<Alg, MODE == kSsGrad>(a, b);
      issue_barrier();
      if (lane == 0) s_model = mrow;
      typename Alg::coef P = ss_pow2<Alg>(mrow.A, __builtin_ctz(K));
#pragma unroll
      for (int i = 0; i < 6; ++i) {
        if (lane == 0) s_tab.pw[i] = P;
        P = Alg::cmul(P, P);
      }
      if (lane == 0) s_tab.pw[6] = P;
#pragma unroll
      for (int r = 1; r < R; r <<= 1) P = Alg::cmul(P, P);
      if (lane == 0) s_tab.pw[7] = P;
      {  // G = A^(kWaves * 64 K R)
        typename Alg::coef G = P;
#pragma unroll
        for (int j = 1; j < kWaves; ++j) G = Alg::cmul(P, G);
        P = G;
      }
#pragma unroll
      for (int j = 0; j < 7; ++j) {
        if (lane == 0) s_tab.gp[j] = P;
        P = Alg::cmul(P, P);
      }
    }
    __syncthreads();  // power tables
    tag = claim_tag(a.claims, a.per_stripe, lane);
    uint64_t *row_status = a.status + b * a.tiles_per_row * St::kStride;
    // The row's entry state.  A zero-phase pass derives it from the row's
    // edge, which only tile 0 needs: tile 0 publishes inclusive states only,
    // so a look-back from a later tile never passes it (the fallback does).
    S virt = Alg::szero();
    if (a.virt_mode == 0) {
      if (a.zi) virt = Alg::load_s(V::load_vec(a.zi + b * V::M));
    } else if (q == 0) {
      virt = ss_filtfilt_entry<Alg>(a, b, lane);
    }
    S yin = virt;
    __syncthreads();  // wave aggregates are in s_wagg
    // exclusive wave prefixes and the tile aggregate (every lane, uniformly)
    S tagg = Alg::szero();
#pragma unroll
    for (int j = 0; j < kWaves; ++j) {
      if (lane == 0) s_wpre[j] = tagg;
      tagg = Alg::affine(s_tab.pw[7], tagg, s_wagg[j]);
    }
    if (q > 0) {
      if (lane == 0) publish(row_status + q * St::kStride + St::kVecWords, tagg, tag);
      if (!ss_lookback<Alg>(row_status, virt, lane, tag, a.spin_limit, s_look, &s_tab, q, yin))
        yin = ss_prefix_fallback<Alg, Sh, REV, MODE == kSsGrad>(kernel_args<SsArgs<Alg>>(), b, q * Sh::kTile, lane,
                                                                virt, &s_tab);
    }
    if (q + 1 < a.tiles_per_row && lane == 0 && !(a.agg_only && q > 0))
      publish(row_status + q * St::kStride, Alg::affine(s_tab.gp[0], yin, tagg), tag);
    if (lane == 0) s_in = yin;
    __syncthreads();  // entry state is in s_in
    return;
  }

  // ================= data waves
  const bool vec = a.vec_ok != 0;
  const E *xrow = a.x + b * T;
  const int64_t seg0 = q * Sh::kTile + int64_t(w) * Sh::kWaveSeg;
  const int sl = ss_scan_lane<REV>(lane);
  // fp32 orders 3-4: the data waves read the model themselves and fold
  // before the power tables are in (the look-back wave's 4 x 4 products take
  // longer than the loads): 52.5 -> 49.1 us forward and 52.9 -> 49.7
  // reversed at order 4 on the C4 shape.  Orders 1-2 (a short table build)
  // and fp64 (register spills at order 4) take the model from LDS.
  constexpr bool kOwnModel = V::M >= 3 && sizeof(E) == 4;
  // The data path, compiled twice: kFull for tiles wholly inside the row
  // with aligned rows (vector loads and stores only, so each round's fold
  // waits for its own loads), and the bounds-checked form.
  auto data_path = [&](auto full_c) {
    constexpr bool kFull = decltype(full_c)::value;
    issue_barrier();  // the look-back wave has issued the model's reads
    SsModel<Alg> mown;
    if constexpr (kOwnModel) mown = ss_model<Alg, MODE == kSsGrad>(a, b);
    int64_t t0s[R];
    E X[R][K];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      t0s[r] = seg0 + int64_t(r) * 64 * K + int64_t(sl) * K;
      ss_load<REV, E, K, kFull>(xrow, t0s[r], T, vec, X[r]);
    }
    // ---- pass 1: every map's matrix part is a known power of A, so only the
    // vector parts are scanned.  Steps past the row's end take a zero input
    // and only touch the aggregate of its last tile, which nobody reads.
    S v[R];
    if constexpr (kOwnModel) {
#pragma unroll
      for (int r = 0; r < R; ++r) v[r] = ss_lane_fold<Alg, K>(mown, X[r]);
    }
    __syncthreads();  // power tables and the model
    // Otherwise the model comes from LDS as wave-uniform values, and the
    // data waves issue no global load but the inputs' before pass 1.
    const SsModel<Alg> m = kOwnModel ? mown : read_lane(s_model, 0);
    S ex[R];
    S tot[R];
    {
      if constexpr (!kOwnModel) {
#pragma unroll
        for (int r = 0; r < R; ++r) v[r] = ss_lane_fold<Alg, K>(m, X[r]);
      }
#pragma unroll
      for (int r = R - kLR; r < R; ++r) {
#pragma unroll
        for (int j = 0; j < K / kEV; ++j) {
          Vec16 t;
#pragma unroll
          for (int i = 0; i < kEV; ++i) t.e[i] = X[r][j * kEV + i];
          s_xin[((w * kLR + r - (R - kLR)) * (K / kEV) + j) * 64 + lane] = t;
        }
      }
      ss_lane_scan<Alg, R, REV>(v, lane, s_tab.pw);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        tot[r] = read_lane(v[r], ss_last_lane<REV>());
        const S prev = shfl_from(v[r], REV ? lane + 1 : lane - 1);
        ex[r] = sl > 0 ? prev : Alg::szero();
      }
    }
    if (lane == 0) {
      S agg = tot[0];
#pragma unroll
      for (int r = 1; r < R; ++r) agg = Alg::affine(s_tab.pw[6], agg, tot[r]);
      s_wagg[w] = agg;
    }
    __syncthreads();  // wave aggregates are in s_wagg
    __syncthreads();  // entry state is in s_in
    // the wave's entry state: A^(64 K R w) s_in + its exclusive prefix
    S st = s_in;
    for (int j = 0; j < w; ++j) st = Alg::affine(s_tab.pw[7], st, Alg::szero());
    st = Alg::sadd(st, s_wpre[w]);

    // ---- pass 2: round r of the wave starts at st[r] (st[r+1] = A^(64 K)
    // st[r] + tot[r]); a lane enters it at A^(K sl) st[r] + ex[r], then
    // y = c . h + d x and the step
    S ent[R];
    ent[0] = st;
#pragma unroll
    for (int r = 1; r < R; ++r) ent[r] = Alg::affine(s_tab.pw[6], ent[r - 1], tot[r - 1]);
    ss_pow_apply<Alg, 6, R>(s_tab.pw, sl, ent);
    // steps per group: plain outputs are written a 16-byte vector at a time
    // (not held for the whole chunk); the state modes group whole state
    // vectors
    constexpr int G = MODE == kSsPlain ? int(16 / sizeof(E)) : ss_state_group<Alg>();
    static_assert(K % G == 0 && G * sizeof(E) % 16 == 0, "groups of whole output vectors");
    const bool vh = a.vec_hs != 0;
    SsGrad<Alg, E> lacc;
    if constexpr (MODE == kSsGrad) {
#pragma unroll
      for (int j = 0; j < SsGrad<Alg>::kN; ++j) lacc.v[j] = E(0);
    }
    const bool want_y = MODE == kSsPlain || MODE == kSsStatesY || (MODE == kSsGrad && a.y);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r >= R - kLR) {
#pragma unroll
        for (int j = 0; j < K / kEV; ++j) {
          const Vec16 t = s_xin[((w * kLR + r - (R - kLR)) * (K / kEV) + j) * 64 + lane];
#pragma unroll
          for (int i = 0; i < kEV; ++i) X[r][j * kEV + i] = t.e[i];
        }
      }
      const S h0 = Alg::sadd(ent[r], ex[r]);
      if constexpr (MODE == kSsPlain && !REV && V::M == 2) {
        if (a.ckpt && t0s[r] < T && t0s[r] % a.ckpt_every == 0)
          reinterpret_cast<S *>(a.ckpt)[b * a.n_ckpt + t0s[r] / a.ckpt_every] = h0;
      }
      SS h = Alg::store_s(h0);
#pragma unroll
      for (int g0 = 0; g0 < K; g0 += G) {
        SS Hg[G];
        E Xg[G];
        E Og[G];
        if constexpr (MODE == kSsGrad) {
          ss_load<REV, SS, G>(reinterpret_cast<const SS *>(a.hs_fwd) + b * T, t0s[r] + g0, T, vh, Hg);
          ss_load<REV, E, G>(a.x_fwd + b * T, t0s[r] + g0, T, vh, Xg);
        }
#pragma unroll
        for (int k2 = 0; k2 < G; ++k2) {
          const int k = g0 + k2;
          if constexpr (kStates) Hg[k2] = h;
          if constexpr (MODE != kSsStates) {
            Og[k2] = fma(m.d, X[r][k], V::dot(m.c, h));
            if constexpr (MODE == kSsGrad) ss_grad_step<Alg>(lacc, h, Hg[k2], Xg[k2], X[r][k]);
          }
          h = Alg::s_affine(m.A, h, V::scale(m.b, X[r][k]));
          if (MODE != kSsStates && a.zf && t0s[r] + k == T - 1) {
            union {
              SS s;
              E e[V::M];
            } u;
            u.s = h;
#pragma unroll
            for (int i = 0; i < V::M; ++i) a.zf[b * V::M + i] = u.e[i];
          }
        }
        if constexpr (kFull && kHLds)
          ss_lds_put<kNVh, REV, K>(s_ht + w * 64 * kNVh, lane, g0, Hg);
        else if constexpr (kStates)
          ss_store<REV, SS, G>(reinterpret_cast<SS *>(a.hs) + b * T, t0s[r] + g0, T, vh, Hg);
        if constexpr (kFull && kYLds)
          ss_lds_put<kNVy, REV, K>(s_yt + w * 64 * kNVy, lane, g0, Og);
        else if (want_y)
          ss_store<REV, E, G, kFull>(a.y + b * T, t0s[r] + g0, T, vec, Og);
      }
      // the round's block, lowest time first
      const int64_t p0 = seg0 + int64_t(r) * 64 * K;  // first scan position of the round
      const int64_t tb = REV ? T - p0 - 64 * K : p0;
      if constexpr (kFull && kHLds)
        lds_flush<kNVh>(reinterpret_cast<uint4 *>(reinterpret_cast<SS *>(a.hs) + b * T + tb),
                           s_ht + w * 64 * kNVh, lane, true);
      if constexpr (kFull && kYLds)
        lds_flush<kNVy>(reinterpret_cast<uint4 *>(a.y + b * T + tb), s_yt + w * 64 * kNVy, lane, want_y);
    }
    if constexpr (MODE == kSsGrad) {
      // the wave's sums, in a fixed order, one partial per (row, tile, wave)
      auto add = [](const SsGrad<Alg> &p, const SsGrad<Alg> &o) {
        SsGrad<Alg> r;
#pragma unroll
        for (int j = 0; j < SsGrad<Alg>::kN; ++j) r.v[j] = p.v[j] + o.v[j];
        return r;
      };
      SsGrad<Alg> gacc;
#pragma unroll
      for (int j = 0; j < SsGrad<Alg>::kN; ++j) gacc.v[j] = up(lacc.v[j]);
      gacc = wave_scan_incl(gacc, lane, add);
      if (lane == 63) {
        auto *dst = a.gpart + ((b * a.tiles_per_row + q) * kWaves + w) * SsGrad<Alg>::kN;
#pragma unroll
        for (int j = 0; j < SsGrad<Alg>::kN; ++j) dst[j] = gacc.v[j];
      }
    }
  };
  // the state modes' full path also needs 16-byte state rows (vec_hs)
  if (vec && (!kStates || a.vec_hs) && (q + 1) * Sh::kTile <= T)
    data_path(std::true_type{});
  else
    data_path(std::false_type{});
}

// ------------------------------------------------------------ coefficient gradients
// Where the sums go: the explicit model's dL/dA, dL/db, dL/dc, dL/dd (each
// nullable; one per row, or one in all for a shared operand), or the
// filter's dL/dfb, dL/dfa by the chain rule through its companion model.
template <typename E>
struct SsGradOut {
  E *gA, *gb, *gc, *gd;
  bool A_sh, b_sh, c_sh, d_sh;
  E *gfb, *gfa;  // filter mode (form != 0)
  const E *fb, *fa;
  int nb, na, form;
  bool f_sh;
  // T == 0: grad_zi = grad_zf (or 0), written here
  E *gzi;
  const E *gzf;
};

constexpr int kSsReduceThreads = 256;

// Row b's sums over its per-wave partials (fixed order): rowsum[b, j].  Each
// thread sums a strided share of the partials for every component, then one
// tree over the block.
template <class Alg>
__global__ __launch_bounds__(kSsReduceThreads) void ss_grad_rows_kernel(
    const typename Wide<typename Alg::elem>::type *gpart, int64_t per_row,
    typename Wide<typename Alg::elem>::type *rowsum) {
  using C = typename Wide<typename Alg::elem>::type;
  constexpr int N = SsGrad<Alg>::kN;
  __shared__ C s[N][kSsReduceThreads];
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  C acc[N];
#pragma unroll
  for (int j = 0; j < N; ++j) acc[j] = 0;
  for (int64_t i = tid; i < per_row; i += kSsReduceThreads) {
    const C *p = gpart + (b * per_row + i) * N;
#pragma unroll
    for (int j = 0; j < N; ++j) acc[j] += p[j];
  }
#pragma unroll
  for (int j = 0; j < N; ++j) s[j][tid] = acc[j];
  __syncthreads();
  for (int h = kSsReduceThreads / 2; h > 0; h >>= 1) {
    if (tid < h) {
#pragma unroll
      for (int j = 0; j < N; ++j) s[j][tid] += s[j][tid + h];
    }
    __syncthreads();
  }
  if (tid < N) rowsum[b * N + tid] = s[tid][0];
}

// dL/dfb, dL/dfa of one filter from its model's sums G (chain rule through
// the companion model of ss_model: TDF-II b = fb[1:] - fb[0] a, A[i][0] =
// -a_i; DF-II c = fb[1:] - fb[0] a, A[0][j] = -a_j; d = fb[0]).
template <class Alg>
__device__ void ss_filter_chain(const typename Wide<typename Alg::elem>::type *Gs, const SsGradOut<typename Alg::elem> &o,
                                const typename Alg::elem *fb, const typename Alg::elem *fa, typename Alg::elem *gfb,
                                typename Alg::elem *gfa) {
  using E = typename Alg::elem;
  using C = typename Wide<E>::type;
  using G = SsGrad<Alg>;
  constexpr int M = G::M;
  const C b0 = C(fb[0]);
  const int vec_at = o.form == 1 ? G::kB : G::kC;  // the vector that carries fb[1:] - fb[0] a
  C g0 = Gs[G::kD];
#pragma unroll
  for (int i = 0; i < M; ++i) {
    const C ai = i < o.na ? C(fa[i]) : C(0);
    const C gv = Gs[vec_at + i];
    g0 -= ai * gv;
    if (i + 1 < o.nb) gfb[i + 1] = E(gv);
    const C gA = o.form == 1 ? Gs[G::kA + i * M] : Gs[G::kA + i];  // A[i][0] or A[0][i]
    if (i < o.na) gfa[i] = E(-gA - b0 * gv);
  }
  gfb[0] = E(g0);
}

// Every output from the row sums: shared operands summed over the rows (a
// tree over the block, fixed order), the filter's chain rule per row or
// once.  One block.
template <class Alg>
__global__ __launch_bounds__(kSsReduceThreads) void ss_grad_finish_kernel(
    const typename Wide<typename Alg::elem>::type *rowsum, int64_t B, int64_t T, SsGradOut<typename Alg::elem> o) {
  using E = typename Alg::elem;
  using C = typename Wide<E>::type;
  using G = SsGrad<Alg>;
  constexpr int M = G::M, N = G::kN;
  __shared__ C s[kSsReduceThreads];
  __shared__ C tot[N];
  const int tid = threadIdx.x;
  if (T == 0 && o.gzi) {
    for (int64_t i = tid; i < B * M; i += kSsReduceThreads) o.gzi[i] = o.gzf ? o.gzf[i] : E(0);
  }
  auto total = [&](int j) {
    C acc = 0;
    for (int64_t b = tid; b < B; b += kSsReduceThreads) acc += rowsum[b * N + j];
    s[tid] = acc;
    __syncthreads();
    for (int h = kSsReduceThreads / 2; h > 0; h >>= 1) {
      if (tid < h) s[tid] += s[tid + h];
      __syncthreads();
    }
    if (tid == 0) tot[j] = s[0];
    __syncthreads();
  };
  if (o.form != 0) {
    if (o.f_sh) {
      for (int j = 0; j < N; ++j) total(j);
      if (tid == 0) ss_filter_chain<Alg>(tot, o, o.fb, o.fa, o.gfb, o.gfa);
    } else {
      for (int64_t b = tid; b < B; b += kSsReduceThreads)
        ss_filter_chain<Alg>(rowsum + b * N, o, o.fb + b * o.nb, o.fa + b * o.na, o.gfb + b * o.nb,
                             o.gfa + b * o.na);
    }
    return;
  }
  struct Part {
    E *dst;
    bool sh;
    int off, n;
  };
  const Part parts[4] = {{o.gA, o.A_sh, G::kA, M * M}, {o.gb, o.b_sh, G::kB, M}, {o.gc, o.c_sh, G::kC, M},
                         {o.gd, o.d_sh, G::kD, 1}};
  for (int p = 0; p < 4; ++p) {
    const Part pt = parts[p];
    if (!pt.dst) continue;
    if (pt.sh) {
      for (int j = 0; j < pt.n; ++j) total(pt.off + j);
      if (tid < pt.n) pt.dst[tid] = E(tot[pt.off + tid]);
      __syncthreads();
    } else {
      for (int64_t i = tid; i < B * pt.n; i += kSsReduceThreads) {
        const int64_t b = i / pt.n;
        pt.dst[i] = E(rowsum[b * N + pt.off + int(i - b * pt.n)]);
      }
    }
  }
}

// ------------------------------------------------------ zero-phase filter backward
// Gradients of y = filtfilt(fb, fa, x) over the padded row ext of N = T + 2e
// samples: pass 1 runs the TDF-II model (A = companion(a)^T, g, c = e0,
// d = b0) from h1[0] = z ext[0] over ext, pass 2 the same model from z
// y1[N-1] over the reversed y1, and y is pass 2's output at the T interior
// samples.  The adjoint model (DF-II of the same b and a: A^T =
// companion(a), input vector e0, output vector g, d = b0) runs twice, each
// time in the opposite direction of its pass:
//  * pass 2's adjoint in ascending time over the upstream gradient padded
//    with zeros: its state stays zero through the front pad; the interior is
//    an ss_kernel launch from a zero state (dL/dy1 there, state lambda_A);
//    the back pad continues from lambda_A with a zero input (dL/dy1 there);
//    its final state dL/dh2[0] adds z . dL/dh2[0] to dL/dy1[N-1] (h2[0] =
//    z y1[N-1]);
//  * pass 1's adjoint in descending time over dL/dy1: the back pad from a
//    zero state (dL/dext there, and the interior's entry state); the
//    interior an ss_kernel launch in reversed time (dL/dx there, state
//    lambda_B); the front pad continues from lambda_B with a zero input
//    (dL/dy1 is zero there: pass 2's adjoint state is) (dL/dext there); its
//    final state dL/dh1[0] adds z . dL/dh1[0] to dL/dext[0];
//  * dL/dext of the pads folds into dL/dx through the pad's index map (the
//    adjoint of F.pad; constant pads hold no x).
// With coefficient gradients every step n of either pass also adds, with
// lambda the adjoint state before the step (dL/d of the state after it), h
// the forward state before it, u its input and gy its upstream gradient,
//     dL/dA += lambda h^T,  dL/dg += lambda u,  dL/db0 += gy u
// (the interiors in the ss_kernel launches' gradient mode, the pads here,
// from the forward states the two passes take through them), the initial
// states add dL/dz = dL/dh1[0] ext[0] + dL/dh2[0] y1[N-1], and z = (I -
// A)^-1 g adds w z^T to dL/dA and w to dL/dg, w = (I - A)^-T dL/dz; the
// filter chain rule maps (A, g, b0) to dL/dfb, dL/dfa.
// The pad pieces run serially per row in double, one thread per row:
// ff_bwd_edge_kernel between the two adjoint launches, ff_bwd_fold_kernel
// after them, a few passes of e steps each (as the forward's entry states).
template <typename E>
struct FfBwdArgs {
  const E *fb, *fa;
  int nb, na;
  int64_t f_stride_b, f_stride_a;  // 0 = shared
  int64_t B, T, e;
  int pad_mode;
  const E *lam_a;  // [B, M] pass 2's adjoint state after the interior
  E *gy1;          // [B, T] dL/dy1 of the interior (pass 1's adjoint input)
  double *edge;    // [B, e] the back pad's dL/dy1, then its dL/dext
  E *entry;        // [B, M] pass 1's adjoint state entering the interior
  const E *lam_b;  // [B, M] pass 1's adjoint state after the interior
  E *gx;           // [B, T]
  // coefficient gradients (coef != 0)
  int coef;
  const E *x;        // [B, T]
  const E *y1;       // [B, T] pass 1's output over the interior
  const E *zf1;      // [B, M] pass 1's state after the interior
  double *work;      // [B, e, 2M + 2] the pad steps' working values (pads longer than kFfPadLds)
  double *gz;        // [B, M] dL/dz of the edge kernel's part
  double *rowsum1;   // [B, kN] pass 1's interior sums (ss_grad_rows_kernel), the total on exit
  double *rowsum2;   // [B, kN] pass 2's interior sums, the back pad's added by the edge kernel
};

// One step of the adjoint model from state s with input u; returns the
// output (o = g . s + b0 u, s' = companion(a) s + e0 u).
template <int M>
__device__ __forceinline__ double ff_adj_step(const FfModel<M> &f, double (&s)[M], double u) {
  double o = f.b0 * u, s0 = u;
#pragma unroll
  for (int i = 0; i < M; ++i) {
    o += f.g[i] * s[i];
    s0 -= f.am[i] * s[i];
  }
#pragma unroll
  for (int i = M - 1; i > 0; --i) s[i] = s[i - 1];
  s[0] = s0;
  return o;
}

// One step of the TDF-II model: h' = A h + g u (A = companion(a)^T; the
// ascending i reads h[i+1] before it changes).
template <int M>
__device__ __forceinline__ void ff_fwd_step(const FfModel<M> &f, double (&h)[M], double u) {
  const double h0 = h[0];
#pragma unroll
  for (int i = 0; i < M; ++i) h[i] = -f.am[i] * h0 + (i + 1 < M ? h[i + 1] : 0.0) + f.g[i] * u;
}

template <int M>
__device__ __forceinline__ double ff_dot_z(const FfModel<M> &f, const double (&s)[M]) {
  double c = 0.0;
#pragma unroll
  for (int i = 0; i < M; ++i) c += f.z[i] * s[i];
  return c;
}

// The model's gradient sums of one step (the SsGrad layout: A row-major, g,
// c (unused: c is e0), b0).
template <int M>
struct FfSums {
  static constexpr int kB = M * M, kD = M * M + 2 * M, kN = M * M + 2 * M + 1;
  double v[kN];
  __device__ __forceinline__ void step(const double (&lam)[M], const double *h, double u, double gy) {
#pragma unroll
    for (int i = 0; i < M; ++i) {
#pragma unroll
      for (int j = 0; j < M; ++j) v[i * M + j] += lam[i] * h[j];
      v[kB + i] += lam[i] * u;
    }
    v[kD] += gy * u;
  }
};

// The per-row pad kernels' working values: for each pad step the forward
// states of both passes, pass 1's output and the adjoint's value (kFfW
// doubles).  Pads of at most kFfPadLds steps live in LDS, one column per
// row (kFfRows rows a block); longer ones in the global work buffer
// ([B, e, kFfW]), where every step would wait on a store's round trip.
constexpr int kFfRows = 32;
constexpr int kFfPadLds = 16;
template <int M>
struct FfPad {
  static constexpr int kW = 2 * M + 2;  // h1 [0, M), h2 [M, 2M), y1 2M, u 2M + 1
};

// Pad-step loops: unrolled over at most EMAX steps (EMAX > 0: the LDS
// path, whose indices are then compile-time) or over e.
template <int EMAX, class F>
__device__ __forceinline__ void ff_up(int64_t e, F &&f) {
  if constexpr (EMAX > 0) {
#pragma unroll
    for (int j = 0; j < EMAX; ++j)
      if (j < e) f(int64_t(j));
  } else {
    for (int64_t j = 0; j < e; ++j) f(j);
  }
}
template <int EMAX, class F>
__device__ __forceinline__ void ff_down(int64_t e, F &&f) {
  if constexpr (EMAX > 0) {
#pragma unroll
    for (int j = EMAX - 1; j >= 0; --j)
      if (j < e) f(int64_t(j));
  } else {
    for (int64_t j = e - 1; j >= 0; --j) f(j);
  }
}

// Between the adjoint launches: pass 2's adjoint over the back pad and its
// edge term, then pass 1's adjoint over the back pad (its dL/dext, the
// fold kernel's input) up to the interior's entry state.  With no pad the
// edge term lands on the interior's last dL/dy1.  With coefficient
// gradients, first the forward states of both passes over the back pad
// (pass 1 from zf1 over the pad's samples, pass 2 from z y1[N-1] back over
// pass 1's outputs there), then both adjoints' sums over it, added to
// rowsum2, and pass 2's part of dL/dz.
template <typename E, int M, int EMAX>
__global__ __launch_bounds__(kFfRows) void ff_bwd_edge_kernel(FfBwdArgs<E> a) {
  constexpr int W = FfPad<M>::kW;
  __shared__ double lds[EMAX > 0 ? EMAX * W : 1][kFfRows];
  const int tid = threadIdx.x;
  const int64_t b = int64_t(blockIdx.x) * kFfRows + tid;
  if (b >= a.B) return;
  const FfModel<M> f = ff_model<M>(a.fb + b * a.f_stride_b, a.nb, a.fa + b * a.f_stride_a, a.na);
  const int64_t T = a.T, e = a.e;
  const bool coef = a.coef != 0;
  const E *xr = coef ? a.x + b * T : nullptr;
  auto w = [&](int64_t j, int k) -> double & {  // the forward values (coefficient gradients only)
    if constexpr (EMAX > 0)
      return lds[j * W + k][tid];
    else
      return a.work[(b * e + j) * W + k];
  };
  double *ub = a.edge + b * e;
  auto u = [&](int64_t j) -> double & {  // dL/dy1 of the back pad, then its dL/dext in ub
    if constexpr (EMAX > 0)
      return lds[j * W + 2 * M + 1][tid];
    else
      return ub[j];
  };
  double ylast = 0.0;
  if (coef) {
    double h[M];
#pragma unroll
    for (int i = 0; i < M; ++i) h[i] = double(a.zf1[b * M + i]);
    ff_up<EMAX>(e, [&](int64_t j) {
      const double xj = double(pad_back(xr, T, a.pad_mode, j));
#pragma unroll
      for (int i = 0; i < M; ++i) w(j, i) = h[i];
      w(j, 2 * M) = h[0] + f.b0 * xj;
      ff_fwd_step(f, h, xj);
    });
    ylast = e > 0 ? w(e - 1, 2 * M) : double(a.y1[b * T + T - 1]);
#pragma unroll
    for (int i = 0; i < M; ++i) h[i] = f.z[i] * ylast;
    ff_down<EMAX>(e, [&](int64_t j) {
#pragma unroll
      for (int i = 0; i < M; ++i) w(j, M + i) = h[i];
      ff_fwd_step(f, h, w(j, 2 * M));
    });
  }
  FfSums<M> acc;
#pragma unroll
  for (int k = 0; k < FfSums<M>::kN; ++k) acc.v[k] = 0.0;
  double s[M], r[M], hj[M];
#pragma unroll
  for (int i = 0; i < M; ++i) {
    s[i] = double(a.lam_a[b * M + i]);
    r[i] = 0.0;
  }
  ff_up<EMAX>(e, [&](int64_t j) {
    if (coef) {
#pragma unroll
      for (int i = 0; i < M; ++i) hj[i] = w(j, M + i);
      acc.step(s, hj, w(j, 2 * M), 0.0);
    }
    u(j) = ff_adj_step(f, s, 0.0);
  });
  const double c = ff_dot_z(f, s);
  if (e > 0) {
    u(e - 1) += c;
  } else {
    E *p = a.gy1 + b * T + (T - 1);
    *p = E(double(*p) + c);
  }
  ff_down<EMAX>(e, [&](int64_t j) {
    const double uj = u(j);
    if (coef) {
#pragma unroll
      for (int i = 0; i < M; ++i) hj[i] = w(j, i);
      acc.step(r, hj, double(pad_back(xr, T, a.pad_mode, j)), uj);
    }
    ub[j] = ff_adj_step(f, r, uj);
  });
#pragma unroll
  for (int i = 0; i < M; ++i) a.entry[b * M + i] = E(r[i]);
  if (coef) {
    double *rs = a.rowsum2 + b * FfSums<M>::kN;
#pragma unroll
    for (int k = 0; k < FfSums<M>::kN; ++k) rs[k] += acc.v[k];
#pragma unroll
    for (int i = 0; i < M; ++i) a.gz[b * M + i] = s[i] * ylast;
  }
}

// After the adjoint launches: pass 1's adjoint over the front pad from
// lambda_B and its edge term, then both pads' dL/dext folded into dL/dx
// (serial per row, so pads that map onto one sample add up in order).  With
// coefficient gradients also pass 1's forward states over the front pad
// (from z ext[0]), the adjoint's sums over it, dL/dz through z = (I -
// A)^-1 g, and the row's total: rowsum1 += rowsum2 + the front pad's sums +
// the steady state's.
template <typename E, int M, int EMAX>
__global__ __launch_bounds__(kFfRows) void ff_bwd_fold_kernel(FfBwdArgs<E> a) {
  constexpr int W = FfPad<M>::kW;
  __shared__ double lds[EMAX > 0 ? EMAX * M : 1][kFfRows];
  const int tid = threadIdx.x;
  const int64_t b = int64_t(blockIdx.x) * kFfRows + tid;
  if (b >= a.B) return;
  const FfModel<M> f = ff_model<M>(a.fb + b * a.f_stride_b, a.nb, a.fa + b * a.f_stride_a, a.na);
  const int64_t T = a.T, e = a.e;
  const bool coef = a.coef != 0;
  const bool to_x = e == 0 || a.pad_mode != kPadConstant;  // pads that hold samples of x
  const bool refl = a.pad_mode == kPadReflect, repl = a.pad_mode == kPadReplicate;
  E *gx = a.gx + b * T;
  const E *xr = coef ? a.x + b * T : nullptr;
  const double *ub = a.edge + b * e;
  auto h1f = [&](int64_t n, int i) -> double & {  // pass 1's states over the front pad
    if constexpr (EMAX > 0)
      return lds[n * M + i][tid];
    else
      return a.work[(b * e + n) * W + i];
  };
  double ext0 = 0.0;
  if (coef) {
    ext0 = double(e > 0 ? pad_front(xr, T, e, a.pad_mode, 0) : xr[0]);
    double h[M];
#pragma unroll
    for (int i = 0; i < M; ++i) h[i] = f.z[i] * ext0;
    ff_up<EMAX>(e, [&](int64_t n) {
#pragma unroll
      for (int i = 0; i < M; ++i) h1f(n, i) = h[i];
      ff_fwd_step(f, h, double(pad_front(xr, T, e, a.pad_mode, n)));
    });
  }
  FfSums<M> acc;
#pragma unroll
  for (int k = 0; k < FfSums<M>::kN; ++k) acc.v[k] = 0.0;
  double r[M], hn[M];
#pragma unroll
  for (int i = 0; i < M; ++i) r[i] = double(a.lam_b[b * M + i]);
  auto add = [&](int64_t i, double v) { gx[i] = E(double(gx[i]) + v); };
  double sf = 0.0, sb = 0.0;  // replicate: everything lands on x[0] and x[T - 1]
  ff_down<EMAX>(e, [&](int64_t n) {  // ext[n] is x[0], x[e - n] (reflect) or x[T - e + n]
    if (coef) {
#pragma unroll
      for (int i = 0; i < M; ++i) hn[i] = h1f(n, i);
      acc.step(r, hn, double(pad_front(xr, T, e, a.pad_mode, n)), 0.0);
    }
    double o = ff_adj_step(f, r, 0.0);
    if (n == 0) o += ff_dot_z(f, r);
    if (repl)
      sf += o;
    else if (to_x)
      add(refl ? e - n : T - e + n, o);
  });
  if (e == 0) add(0, ff_dot_z(f, r));  // ext is x
  for (int64_t j = 0; j < e; ++j) {  // ext[T + e + j]
    if (repl)
      sb += ub[j];
    else if (to_x)
      add(refl ? T - 2 - j : j, ub[j]);
  }
  if (repl && e > 0) {
    add(0, sf);
    add(T - 1, sb);
  }
  if (!coef) return;
  // dL/dz, then w = (I - companion(a))^-1 dL/dz: rows 1.. give w_i = w_0 +
  // p_i with p_i = sum_{k=1..i} gz_k, row 0 w_0 (1 + sum a) = gz_0 - sum a_i p_i
  double gz[M], p[M], wv[M];
  double sa = 1.0, ap = 0.0;
#pragma unroll
  for (int i = 0; i < M; ++i) {
    gz[i] = a.gz[b * M + i] + r[i] * ext0;
    p[i] = i == 0 ? 0.0 : p[i - 1] + gz[i];
    sa += f.am[i];
    ap += f.am[i] * p[i];
  }
  const double w0 = (gz[0] - ap) / sa;
#pragma unroll
  for (int i = 0; i < M; ++i) {
    wv[i] = w0 + p[i];
#pragma unroll
    for (int j = 0; j < M; ++j) acc.v[i * M + j] += wv[i] * f.z[j];
    acc.v[FfSums<M>::kB + i] += wv[i];
  }
  double *rs = a.rowsum1 + b * FfSums<M>::kN;
  const double *r2 = a.rowsum2 + b * FfSums<M>::kN;
#pragma unroll
  for (int k = 0; k < FfSums<M>::kN; ++k) rs[k] += r2[k] + acc.v[k];
}

}  // namespace phs
