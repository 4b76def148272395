// Fused single-input, single-output LPV (time-varying) state space of order
// M <= 4 in one pass (philtorch/lpv/ssm.py:337-581: state_space with a 2D
// input, B an M-vector per row and/or per step or absent, C an M-vector per
// row and/or per step or out_idx, D per row and/or per step or absent; the
// glue of lpv/ssm.py:413-577 folded into the scan):
//     h[0] = zi,  y[t] = c[t] . h[t] + d[t] x[t],  h[t+1] = A[t] h[t] + b[t] x[t],
//     zf = h[T]
// Per step the kernel reads A[t], x[t] and whichever of b[t], c[t], d[t] vary
// along time, and writes y[t]; the reference route writes and reads B x, the
// state sequence, its shifted copy, C h and D x.
//
// The scan is the generic one (phs_scan.hpp) in its time-varying mode: a lane
// folds its K steps (A[t], b[t] x[t]) into a map, wave scans chain the lanes,
// a look-back wave resolves the tile's entry state over the row's status
// words, and pass 2 re-runs the steps from each lane's entry state, writing
// c[t] . h + d[t] x[t] instead of h.  A reversed mode runs the model
// backwards in time: the gradients w.r.t. x and zi are that mode on the
// adjoint model.  Those of A, b, c, d take two launches, as for the LTI
// model (phs_ss.hpp): the forward again writing its states (kSsStates),
// then the adjoint pass (kSsGrad), which at every step writes
//     dL/dA[t] = lambda[t+1] h[t]^T, dL/db[t] = lambda[t+1] x[t],
//     dL/dc[t] = g[t] h[t],          dL/dd[t] = g[t] x[t]
// for the operands that vary along time (into a per-row scratch where the
// rows share them, summed over the rows afterwards) and sums them per wave
// for those constant in time.
#pragma once

#include "phs_ss.hpp"

namespace phs {

// A per-row and/or per-step operand: element (row, t, i) at
// p + row * row_stride + t * t_stride + i (a stride 0 shares that axis).
template <typename E>
struct LpvOperand {
  const E *p;
  int64_t row_stride, t_stride;
};

template <class Alg>
struct LpvSsArgs {
  using E = typename Alg::elem;
  const E *A;            // [rows, T, M, M]
  int64_t A_row_stride;  // elements between rows (0 = shared)
  int A_trans;           // read each step's matrix transposed (the adjoint model's A[t]^T)
  LpvOperand<E> bv;      // [., ., M]; p nullptr: the input enters state in_idx
  LpvOperand<E> cv;      // [., ., M]; p nullptr: y is state out_idx
  LpvOperand<E> d;       // [., .]; p nullptr: no feedthrough
  int out_idx, in_idx;  // in_idx: read in kSsGrad only (the other modes take 0)
  const E *zi;  // [B, M]; nullptr: zeros
  const E *x;   // [B, T]
  E *y;         // [B, T]
  E *zf;        // [B, M]; nullable
  // kSsStates: the state before every step [B, T, M] (no y); kSsGrad: the
  // forward's states and input, the per-(row, step) gradients of the
  // operands that vary along time ([B, T, M*M], [B, T, M], [B, T, M],
  // [B, T]; each nullable; dL/dA[t] written transposed with gA_trans, for
  // a forward that read A transposed) and the per-wave sums of b, c, d where
  // they are constant in time ([B, tiles, kWaves, SsGrad::kN])
  E *hs;
  const E *hs_fwd, *x_fwd;
  int vec_hs;
  E *gA_step, *gb_step, *gc_step, *gd_step;
  int gA_trans;
  int sum_b, sum_c, sum_d;
  typename Wide<E>::type *gpart;
  int64_t B, T_len, tiles_per_row;
  uint64_t b_magic;  // tile id -> row by multiply and shift (row_split)
  unsigned b_shift;
  unsigned long long *claims;
  unsigned tiles, per_stripe, spin_limit;
  unsigned agg_only;  // testing: tiles after a row's first publish no inclusive state
  uint64_t *status;
  int vec_ok;
};

// 3 data waves and a look-back wave; the time-varying scan's steps per lane
// and rounds (Shape<Alg, true>), except order 4: there that is one step per
// lane, so six 4x4 map compositions of the wave scan per step; 4 steps in
// one round measured 0.49 against 1.03 ms at the C4 shape (order 3 is
// faster with its own 4 x 2: 0.22 against 0.29 ms).
template <class Alg>
struct LpvSsShape {
  static constexpr int kM = int(sizeof(typename Alg::s_state) / sizeof(typename Alg::elem));
  static constexpr int kWaves = 3;
  static constexpr int kThreads = 64 * (kWaves + 1);
  static constexpr int K = kM == 4 ? 4 : Shape<Alg, true>::K;
  static constexpr int R = kM == 4 ? 1 : Shape<Alg, true>::R;
  static constexpr int kTile = kWaves * 64 * K * R;
};

// K items of a row in scan order from scan position s0: forward, position s
// is time s; reversed (REV), time T-1-s, so the chunk is the K items below
// T - s0 read in descending time.  Positions past the row read `fill`.
template <bool REV, typename X, int K>
__device__ __forceinline__ void lpv_load(const X *row, int64_t s0, int64_t T, bool vec, X (&out)[K], const X fill) {
  constexpr bool kVec = (K * sizeof(X)) % 16 == 0;
  if constexpr (!REV) {
    if constexpr (kVec) {
      load_chunk<X, K>(row, s0, T, vec, out, fill);
    } else {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        if (s0 + k < T)
          out[k] = row[s0 + k];
        else
          out[k] = fill;
      }
    }
  } else {
    const int64_t base = T - s0 - K;
    if (kVec && vec && base >= 0) {
      X tmp[K];
      if constexpr (kVec) load_chunk<X, K>(row, base, T, true, tmp, fill);
#pragma unroll
      for (int k = 0; k < K; ++k) out[k] = tmp[K - 1 - k];
    } else {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int64_t t = T - 1 - s0 - k;
        if (t >= 0)
          out[k] = row[t];
        else
          out[k] = fill;
      }
    }
  }
}

template <bool REV, typename X, int K>
__device__ __forceinline__ void lpv_store(X *row, int64_t s0, int64_t T, bool vec, const X (&v)[K]) {
  constexpr bool kVec = (K * sizeof(X)) % 16 == 0;
  if constexpr (!REV) {
    if constexpr (kVec) {
      store_chunk<X, K>(row, s0, T, vec, v);
    } else {
#pragma unroll
      for (int k = 0; k < K; ++k)
        if (s0 + k < T) row[s0 + k] = v[k];
    }
  } else {
    const int64_t base = T - s0 - K;
    if (kVec && vec && base >= 0) {
      X tmp[K];
#pragma unroll
      for (int k = 0; k < K; ++k) tmp[k] = v[K - 1 - k];
      if constexpr (kVec) store_chunk<X, K>(row, base, T, true, tmp);
    } else {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int64_t t = T - 1 - s0 - k;
        if (t >= 0) row[t] = v[k];
      }
    }
  }
}

// Time of scan position s (clamped into the row: positions past it carry a
// zero input and coefficient, and their outputs are not stored).
template <bool REV>
__device__ __forceinline__ int64_t lpv_time(int64_t s, int64_t T) {
  const int64_t t = REV ? T - 1 - s : s;
  return t < 0 ? 0 : (t >= T ? T - 1 : t);
}

// b[t] x[t] for the K steps from scan position s0 (b absent: x[t] into
// state in_idx, 0 but in the adjoint of a model with its output state
// selected).
template <class Alg, bool REV, int K>
__device__ __forceinline__ void lpv_inputs(const LpvSsArgs<Alg> &a, int64_t b, int64_t s0, const typename Alg::elem (&u)[K],
                                           typename Alg::s_state (&X)[K], int in_idx) {
  using V = SsView<Alg>;
  using E = typename Alg::elem;
  // (one uniform branch for the chunk, no per-step select between a load
  // and a constant)
  if (a.bv.p) {
    const E *bp = a.bv.p + b * a.bv.row_stride;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int64_t t = lpv_time<REV>(s0 + k, a.T_len);
      X[k] = V::scale(V::load_vec(bp + t * a.bv.t_stride), u[k]);
    }
  } else {
    const typename Alg::s_state e = V::unit(in_idx);
#pragma unroll
    for (int k = 0; k < K; ++k) X[k] = V::scale(e, u[k]);
  }
}

// One step of the adjoint pass's coefficient gradients at time t of row b
// (valid: t inside the row): lambda = dL/dh[t+1] (the adjoint state before
// the step), g = dL/dy[t], hf = h[t], xf = x[t].
template <class Alg>
__device__ __forceinline__ void lpv_grad_step(const LpvSsArgs<Alg> &a, int64_t b, int64_t t, bool valid,
                                              const typename Alg::s_state &lambda, typename Alg::elem g,
                                              const typename Alg::s_state &hf, typename Alg::elem xf,
                                              SsGrad<Alg, typename Alg::elem> &acc) {
  using E = typename Alg::elem;
  using G = SsGrad<Alg, E>;
  constexpr int M = G::M;
  union {
    typename Alg::s_state s;
    E e[M];
  } ul, uh;
  ul.s = lambda;
  uh.s = hf;
  const int64_t rt = b * a.T_len + t;
  if (valid && a.gA_step) {
    union {
      typename Alg::s_coef s;
      E e[M * M];
    } u;
#pragma unroll
    for (int i = 0; i < M; ++i)
#pragma unroll
      for (int j = 0; j < M; ++j) u.e[i * M + j] = a.gA_trans ? uh.e[i] * ul.e[j] : ul.e[i] * uh.e[j];
    reinterpret_cast<typename Alg::s_coef *>(a.gA_step)[rt] = u.s;
  }
  if (valid && a.gb_step) {
#pragma unroll
    for (int i = 0; i < M; ++i) a.gb_step[rt * M + i] = ul.e[i] * xf;
  }
  if (valid && a.gc_step) {
#pragma unroll
    for (int i = 0; i < M; ++i) a.gc_step[rt * M + i] = g * uh.e[i];
  }
  if (valid && a.gd_step) a.gd_step[rt] = g * xf;
  if (a.sum_b) {
#pragma unroll
    for (int i = 0; i < M; ++i) acc.v[G::kB + i] = fma(ul.e[i], xf, acc.v[G::kB + i]);
  }
  if (a.sum_c) {
#pragma unroll
    for (int i = 0; i < M; ++i) acc.v[G::kC + i] = fma(g, uh.e[i], acc.v[G::kC + i]);
  }
  if (a.sum_d) acc.v[G::kD] = fma(g, xf, acc.v[G::kD]);
}

// State entering tile position `span` of a row, folded from the inputs (the
// look-back's bounded-wait fallback; out of line, cold).
template <class Alg, bool REV>
__device__ __noinline__ typename Alg::state lpv_prefix_fallback(const LpvSsArgs<Alg> *ap, int64_t b, int64_t span,
                                                               int lane, typename Alg::state virt, int in_idx) {
  const LpvSsArgs<Alg> &a = *ap;
  using E = typename Alg::elem;
  using SC = typename Alg::s_coef;
  using SS = typename Alg::s_state;
  using M = Map<Alg>;
  constexpr int K = LpvSsShape<Alg>::K;
  auto op = [](const M &p, const M &q) { return compose<Alg>(p, q); };
  const SC *crow = reinterpret_cast<const SC *>(a.A + b * a.A_row_stride);
  const E *xrow = a.x + b * a.T_len;
  const SC dummy = Alg::s_czero();
  M acc = map_identity<Alg>();
  for (int64_t off = 0; off < span; off += 64 * K) {
    const int64_t c0 = off + int64_t(lane) * K;
    E u[K];
    SS xs[K];
    SC cs[K];
    lpv_load<REV, E, K>(xrow, c0, a.T_len, a.vec_ok != 0, u, E(0));
    lpv_load<REV, SC, K>(crow, c0, a.T_len, a.vec_ok != 0, cs, Alg::s_czero());
    if (a.A_trans) {
#pragma unroll
      for (int k = 0; k < K; ++k) cs[k] = Alg::s_adjoint(cs[k]);  // real: the transpose
    }
    lpv_inputs<Alg, REV, K>(a, b, c0, u, xs, in_idx);
    M m = lane_map<Alg, true, false, K>(cs, xs, dummy);
    m = wave_scan_incl(m, lane, op);
    acc = compose<Alg>(acc, read_lane(m, 63));
  }
  return apply<Alg>(acc, virt);
}

// REV runs the model backwards in time: scan position s is time T-1-s (zi
// the state before the last sample, zf after the first), the form of the
// adjoint pass.  MODE as ss_kernel's.
template <class Alg, bool REV, int MODE>
__global__ __launch_bounds__(LpvSsShape<Alg>::kThreads, 2) void lpv_ss_kernel(LpvSsArgs<Alg> a) {
  using E = typename Alg::elem;
  using S = typename Alg::state;
  using SC = typename Alg::s_coef;
  using SS = typename Alg::s_state;
  using M = Map<Alg>;
  using V = SsView<Alg>;
  using Sh = LpvSsShape<Alg>;
  using St = StatusShape<Alg>;
  constexpr int K = Sh::K, R = Sh::R, kWaves = Sh::kWaves;

  __shared__ M s_wagg[kWaves];
  __shared__ M s_wpre[kWaves];
  __shared__ S s_in;
  __shared__ unsigned s_id, s_tag;
  __shared__ uint64_t s_look[St::kLookWords];

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
  const bool vec = a.vec_ok != 0;
  auto op = [](const M &p, const M &q2) { return compose<Alg>(p, q2); };

  if (w == kWaves) {
    // ================= look-back wave
    tag = claim_tag(a.claims, a.per_stripe, lane);
    uint64_t *row_status = a.status + b * a.tiles_per_row * St::kStride;
    const S virt = a.zi ? Alg::load_s(V::load_vec(a.zi + b * V::M)) : Alg::szero();
    __syncthreads();  // wave aggregates are in s_wagg
    M v = lane < kWaves ? s_wagg[lane] : map_identity<Alg>();
    v = wave_scan_incl(v, lane, op);
    const M wex = wave_shift_up(v, lane, map_identity<Alg>());
    if (lane < kWaves) s_wpre[lane] = wex;
    const M tagg = read_lane(v, kWaves - 1);
    S yin = virt;
    if (q > 0) {
      if (lane == 0) publish(row_status + q * St::kStride + St::kIncWords, tagg, tag);
      Lookback<Alg> lb = lookback_start<Alg>(q);
      if (!lookback<Alg>(row_status, virt, lane, tag, a.spin_limit, s_look, lb, yin))
        yin = lpv_prefix_fallback<Alg, REV>(kernel_args<LpvSsArgs<Alg>>(), b, q * Sh::kTile, lane, virt,
                                            MODE == kSsGrad ? a.in_idx : 0);
    }
    if (q + 1 < a.tiles_per_row && lane == 0 && !(a.agg_only && q > 0))
      publish(row_status + q * St::kStride, apply<Alg>(tagg, yin), tag);
    if (lane == 0) s_in = yin;
    __syncthreads();  // entry state is in s_in
    return;
  }

  // ================= data waves
  const SC *crow = reinterpret_cast<const SC *>(a.A + b * a.A_row_stride);
  const E *xrow = a.x + b * T;
  const int64_t seg0 = q * Sh::kTile + int64_t(w) * 64 * K * R;
  auto chunk0 = [&](int r) -> int64_t { return seg0 + int64_t(r) * 64 * K + int64_t(lane) * K; };
  const SC dummy = Alg::s_czero();
  E U[R][K];
  SC A[R][K];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    lpv_load<REV, E, K>(xrow, chunk0(r), T, vec, U[r], E(0));
    lpv_load<REV, SC, K>(crow, chunk0(r), T, vec, A[r], Alg::s_czero());
    if (a.A_trans) {
#pragma unroll
      for (int k = 0; k < K; ++k) A[r][k] = Alg::s_adjoint(A[r][k]);  // real: the transpose
    }
  }

  // ---- pass 1: lane maps of (A[t], b[t] x[t]), wave scans, round chaining.
  // Steps past the row's end take a zero coefficient and input and only
  // touch the aggregate of its last tile, which nobody reads.
  M Ex[R];
  M carry = map_identity<Alg>();
  SS X[R][K];  // b[t] x[t], kept for pass 2 (b is read once)
#pragma unroll
  for (int r = 0; r < R; ++r) {
    lpv_inputs<Alg, REV, K>(a, b, chunk0(r), U[r], X[r], MODE == kSsGrad ? a.in_idx : 0);
    M m = lane_map<Alg, true, false, K>(A[r], X[r], dummy);
    m = wave_scan_incl(m, lane, op);
    const M ex = wave_shift_up(m, lane, map_identity<Alg>());
    const M tot = read_lane(m, 63);
    Ex[r] = compose<Alg>(carry, ex);
    carry = compose<Alg>(carry, tot);
  }
  if (lane == 0) s_wagg[w] = carry;
  __syncthreads();  // wave aggregates are in s_wagg
  __syncthreads();  // entry state is in s_in
  const S hw = apply<Alg>(s_wpre[w], s_in);

  // ---- pass 2: y = c[t] . h + d[t] x[t], then the step
  const E *cp = a.cv.p ? a.cv.p + b * a.cv.row_stride : nullptr;
  const E *dp = a.d.p ? a.d.p + b * a.d.row_stride : nullptr;
  const SS c_fixed = V::unit(a.out_idx);
  const bool vh = a.vec_hs != 0;
  SsGrad<Alg, E> lacc;
  if constexpr (MODE == kSsGrad) {
#pragma unroll
    for (int j = 0; j < SsGrad<Alg>::kN; ++j) lacc.v[j] = E(0);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t t0 = chunk0(r);
    SS h = Alg::store_s(apply<Alg>(Ex[r], hw));
    SS Hf[K];
    E Xf[K];
    if constexpr (MODE == kSsGrad) {
      lpv_load<REV, SS, K>(reinterpret_cast<const SS *>(a.hs_fwd) + b * T, t0, T, vh, Hf, SS{});
      lpv_load<REV, E, K>(a.x_fwd + b * T, t0, T, vh, Xf, E(0));
    }
    E O[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int64_t t = lpv_time<REV>(t0 + k, T);
      if constexpr (MODE == kSsStates || MODE == kSsStatesY) Hf[k] = h;
      if constexpr (MODE != kSsStates) {
        const SS c = cp ? V::load_vec(cp + t * a.cv.t_stride) : c_fixed;
        const E dv = dp ? dp[t * a.d.t_stride] : E(0);
        O[k] = fma(dv, U[r][k], V::dot(c, h));
        if constexpr (MODE == kSsGrad) lpv_grad_step<Alg>(a, b, t, t0 + k < T, h, U[r][k], Hf[k], Xf[k], lacc);
      }
      h = Alg::s_affine(A[r][k], h, X[r][k]);
      if (MODE != kSsStates && a.zf && t0 + k == T - 1) {
        union {
          SS s;
          E e[V::M];
        } zu;
        zu.s = h;
#pragma unroll
        for (int i = 0; i < V::M; ++i) a.zf[b * V::M + i] = zu.e[i];
      }
    }
    if constexpr (MODE == kSsStates || MODE == kSsStatesY)
      lpv_store<REV, SS, K>(reinterpret_cast<SS *>(a.hs) + b * T, t0, T, vh, Hf);
    if constexpr (MODE == kSsPlain || MODE == kSsStatesY)
      lpv_store<REV, E, K>(a.y + b * T, t0, T, vec, O);
    else if (MODE == kSsGrad && a.y)
      lpv_store<REV, E, K>(a.y + b * T, t0, T, vec, O);
  }
  if constexpr (MODE == kSsGrad) {
    if (a.gpart) {  // the wave's sums of the operands constant in time
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
  }
}

// dst[i] = sum over the rows of src[row, i] (i < n), in row order, for the
// per-step gradients of an operand the rows share.
template <typename E>
__global__ __launch_bounds__(256) void lpv_grad_batch_kernel(const E *src, int64_t rows, int64_t n, E *dst) {
  using C = typename Wide<E>::type;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256) {
    C acc = 0;
    for (int64_t r = 0; r < rows; ++r) acc += up(src[r * n + i]);
    dst[i] = down<E>(acc);
  }
}

}  // namespace phs
