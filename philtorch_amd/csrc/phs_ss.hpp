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
// of the M^3 of composing maps.  Forward only: the gradient is the composite
// on the native recurrence ops.
#pragma once

#include "phs_scan.hpp"

namespace phs {

template <class Alg>
struct SsArgs {
  using E = typename Alg::elem;
  const E *A;         // [rows, M, M] row-major
  int64_t A_stride;   // elements between rows (0 = shared)
  const E *bv;        // [rows, M]; nullptr: the input enters state 0
  int64_t b_stride;
  const E *cv;        // [rows, M]; nullptr: y is state out_idx
  int64_t c_stride;
  const E *d;         // [rows]; nullptr: no feedthrough
  int64_t d_stride;
  int out_idx;
  const E *zi;        // [B, M]; nullptr: zeros
  const E *x;         // [B, T]
  E *y;               // [B, T]
  E *zf;              // [B, M]; nullable
  int64_t B, T_len, tiles_per_row;
  unsigned long long *claims;
  unsigned tiles, per_stripe, spin_limit;
  uint64_t *status;
  int vec_ok;
};

// 3 data waves and a look-back wave; 2 rounds of two 16-byte vectors of
// inputs per lane (8 fp32 or 4 fp64 steps).
template <class Alg>
struct SsShape {
  using E = typename Alg::elem;
  static constexpr int kWaves = 3;
  static constexpr int kThreads = 64 * (kWaves + 1);
  static constexpr int K = int(32 / sizeof(E));
  static constexpr int R = 2;
  static constexpr int kWaveSeg = 64 * K * R;
  static constexpr int kTile = kWaves * kWaveSeg;
  static_assert((K & (K - 1)) == 0, "K is a power of two (the lane matrix is A^K by squaring)");
};

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

template <class Alg>
__device__ __forceinline__ SsModel<Alg> ss_model(const SsArgs<Alg> &a, int64_t row) {
  using V = SsView<Alg>;
  using E = typename Alg::elem;
  SsModel<Alg> m;
  m.A = V::load_mat(a.A + row * a.A_stride);
  m.b = a.bv ? V::load_vec(a.bv + row * a.b_stride) : V::unit(0);
  m.c = a.cv ? V::load_vec(a.cv + row * a.c_stride) : V::unit(a.out_idx);
  m.d = a.d ? a.d[row * a.d_stride] : E(0);
  return m;
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

// State entering scan position `span` of a row, folded straight from the
// inputs (the look-back's bounded-wait fallback; out of line, cold).
template <class Alg, class Sh>
__device__ __noinline__ typename Alg::state ss_prefix_fallback(SsArgs<Alg> a, int64_t b, int64_t span, int lane,
                                                              typename Alg::state virt) {
  using E = typename Alg::elem;
  using M = Map<Alg>;
  constexpr int K = Sh::K;
  const SsModel<Alg> m = ss_model<Alg>(a, b);
  const typename Alg::coef AK = ss_pow2<Alg>(m.A, __builtin_ctz(K));
  auto op = [](const M &p, const M &q) { return compose<Alg>(p, q); };
  const E *xrow = a.x + b * a.T_len;
  M acc = map_identity<Alg>();
  for (int64_t off = 0; off < span; off += 64 * K) {
    E xs[K];
    load_chunk<E, K>(xrow, off + int64_t(lane) * K, a.T_len, a.vec_ok != 0, xs, E(0));
    M v = wave_scan_incl(M{AK, ss_lane_fold<Alg, K>(m, xs)}, lane, op);
    acc = compose<Alg>(acc, read_lane(v, 63));
  }
  return apply<Alg>(acc, virt);
}

// At least two waves per SIMD (two workgroups per CU): order 4 otherwise
// takes 315 VGPRs, mostly the look-back wave's 4x4 maps, and holds one tile
// per CU.
template <class Alg>
__global__ __launch_bounds__(SsShape<Alg>::kThreads, 2) void ss_kernel(SsArgs<Alg> a) {
  using E = typename Alg::elem;
  using S = typename Alg::state;
  using SS = typename Alg::s_state;
  using M = Map<Alg>;
  using V = SsView<Alg>;
  using Sh = SsShape<Alg>;
  using St = StatusShape<Alg>;
  constexpr int K = Sh::K, R = Sh::R, kWaves = Sh::kWaves;

  __shared__ M s_wagg[kWaves];
  __shared__ M s_wpre[kWaves];
  __shared__ S s_in;
  __shared__ unsigned s_id, s_tag;
  __shared__ uint64_t s_look[St::kLookWords];
  // matrix parts, all powers of A: s_pw[i] = A^(K 2^i) for the lane scan
  // (i < 6), s_pw[6] = A^(64 K) between rounds, s_pw[7] = A^(64 K R) per wave
  __shared__ typename Alg::coef s_pw[8];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (tid == 0) claim_tile(a.claims, a.per_stripe, s_id, s_tag);
  __syncthreads();
  if (s_id >= a.tiles) return;  // padding of the last stripe round
  const int64_t id = s_id;
  const unsigned tag = s_tag;
  const int64_t q = id / a.B;  // tile position along the row
  const int64_t b = id - q * a.B;
  const int64_t T = a.T_len;
  auto op = [](const M &p, const M &o) { return compose<Alg>(p, o); };

  if (w == kWaves) {
    // ================= look-back wave
    {
      typename Alg::coef P = ss_pow2<Alg>(SsView<Alg>::load_mat(a.A + b * a.A_stride), __builtin_ctz(K));
#pragma unroll
      for (int i = 0; i < 6; ++i) {
        if (lane == 0) s_pw[i] = P;
        P = Alg::cmul(P, P);
      }
      if (lane == 0) s_pw[6] = P;
#pragma unroll
      for (int r = 1; r < R; r <<= 1) P = Alg::cmul(P, P);
      if (lane == 0) s_pw[7] = P;
    }
    __syncthreads();  // power table
    uint64_t *row_status = a.status + b * a.tiles_per_row * St::kStride;
    const S virt = a.zi ? Alg::load_s(V::load_vec(a.zi + b * V::M)) : Alg::szero();
    S yin = virt;
    __syncthreads();  // wave aggregates are in s_wagg
    M v = lane < kWaves ? s_wagg[lane] : map_identity<Alg>();
    v = wave_scan_incl(v, lane, op);
    const M wex = wave_shift_up(v, lane, map_identity<Alg>());
    if (lane < kWaves) s_wpre[lane] = wex;
    const M tagg = read_lane(v, kWaves - 1);
    if (q > 0) {
      if (lane == 0) publish(row_status + q * St::kStride + St::kIncWords, tagg, tag);
      Lookback<Alg> lb = lookback_start<Alg>(q);
      if (!lookback<Alg>(row_status, virt, lane, tag, a.spin_limit, s_look, lb, yin))
        yin = ss_prefix_fallback<Alg, Sh>(a, b, q * Sh::kTile, lane, virt);
    }
    if (q + 1 < a.tiles_per_row && lane == 0) publish(row_status + q * St::kStride, apply<Alg>(tagg, yin), tag);
    if (lane == 0) s_in = yin;
    __syncthreads();  // entry state is in s_in
    return;
  }

  // ================= data waves
  const SsModel<Alg> m = ss_model<Alg>(a, b);
  const bool vec = a.vec_ok != 0;
  const E *xrow = a.x + b * T;
  const int64_t seg0 = q * Sh::kTile + int64_t(w) * Sh::kWaveSeg;
  int64_t t0s[R];
  E X[R][K];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    t0s[r] = seg0 + int64_t(r) * 64 * K + int64_t(lane) * K;
    load_chunk<E, K>(xrow, t0s[r], T, vec, X[r], E(0));
  }
  __syncthreads();  // power table

  // ---- pass 1: every map's matrix part is a known power of A, so only the
  // vector parts are scanned (Kogge-Stone over the lanes, multiplier
  // A^(K 2^i) at level i).  Steps past the row's end take a zero input and
  // only touch the aggregate of its last tile, which nobody reads.
  S ex[R], tot[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    S v = ss_lane_fold<Alg, K>(m, X[r]);
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      const int d = 1 << i;
      const S o = shfl_from(v, lane - d);
      if (lane >= d) v = Alg::affine(s_pw[i], o, v);
    }
    tot[r] = read_lane(v, 63);
    const S prev = shfl_from(v, lane - 1);
    ex[r] = lane > 0 ? prev : Alg::szero();
  }
  if (lane == 0) {
    S agg = tot[0];
#pragma unroll
    for (int r = 1; r < R; ++r) agg = Alg::affine(s_pw[6], agg, tot[r]);
    s_wagg[w] = M{s_pw[7], agg};
  }
  __syncthreads();  // wave aggregates are in s_wagg
  __syncthreads();  // entry state is in s_in
  S st = apply<Alg>(s_wpre[w], s_in);

  // ---- pass 2: a lane enters round r at A^(K lane) st + ex, then
  // y = c . h + d x and the step
  E *yrow = a.y + b * T;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    S e = st;
#pragma unroll
    for (int i = 0; i < 6; ++i)
      if ((lane >> i) & 1) e = Alg::affine(s_pw[i], e, Alg::szero());
    SS h = Alg::store_s(Alg::sadd(e, ex[r]));
    E O[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      O[k] = fma(m.d, X[r][k], V::dot(m.c, h));
      h = Alg::s_affine(m.A, h, V::scale(m.b, X[r][k]));
      if (a.zf && t0s[r] + k == T - 1) {
        union {
          SS s;
          E e[V::M];
        } u;
        u.s = h;
#pragma unroll
        for (int i = 0; i < V::M; ++i) a.zf[b * V::M + i] = u.e[i];
      }
    }
    store_chunk<E, K>(yrow, t0s[r], T, vec, O);
    st = Alg::affine(s_pw[6], st, tot[r]);
  }
}

}  // namespace phs
