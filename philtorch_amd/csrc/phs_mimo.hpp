// Fused multi-input, multi-output LTI state space of order M <= 4 with up to
// four inputs and four outputs per step, in one pass (philtorch/lti/ssm.py:
// 386-589: state_space with a 3D input (batch, time, features), B an M x F
// matrix, C a P x M matrix, D a P x F matrix, each per row or shared; the
// glue of lti/ssm.py:467-471, 493-506 and _ssm_C_D :513-589 folded into the
// scan):
//     h[0] = zi,  y[t] = C h[t] + D x[t],  h[t+1] = A h[t] + B x[t],  zf = h[T]
// x is [rows, T, F] and y [rows, T, P], both with the features innermost.
// Per step F inputs and P outputs move; the reference route writes and reads
// B x, the state sequence, its shifted copy, C h and D x.
//
// The decomposition and the look-back are the LTI state space's
// (phs_ss.hpp): a lane folds its K steps of B x[t] from a zero state in
// compute precision, the data waves scan these vectors against a table of
// A^(K 2^i) in LDS (every map's matrix part is a known power of A, so a level
// is M^2 work on a vector, not M^3 on a map), a look-back wave resolves the
// tile's entry state over vector status words, and pass 2 re-runs the steps
// from each lane's entry state, writing C h + D x.  F and P are arguments, not template parameters: a wave stages
// its span of x through LDS as F planes of one feature each (a lane then
// reads its K steps of feature f at a fixed offset), and its outputs leave
// through P planes the same way, so the global side of both moves is the
// span's contiguous block, one element per lane and instruction.  The
// reversed mode (REV) runs the model backwards in time: the gradients w.r.t.
// x and zi are that mode on the adjoint model (A^T, input matrix C^T, output
// matrix B^T, feedthrough D^T); with C = I and no D the output is the state
// before every step, which the coefficient gradients reduce against.
#pragma once

#include "phs_lpvss.hpp"

namespace phs {

// Largest F and P of a call (the register arrays of the model and of a
// lane's per-step inputs and outputs are this wide).
constexpr int kMimoMaxIO = 4;

template <class Alg>
struct MimoArgs {
  using E = typename Alg::elem;
  const E *A;  // [rows, M, M] row-major; time-varying (lpv_mimo_kernel): [rows, T, M, M]
  int64_t A_stride;  // elements between rows (0 = shared)
  int A_trans;       // time-varying: read each step's matrix transposed (the adjoint model's A[t]^T)
  int A_vec;         // time-varying: a row's matrices lie in whole 16-byte vectors
  const E *Bm;  // [rows, M, F]
  int64_t b_stride;
  const E *Cm;  // [rows, P, M]
  int64_t c_stride;
  const E *Dm;  // [rows, P, F]; nullptr: no feedthrough
  int64_t d_stride;
  int F, P;
  uint64_t f_magic, p_magic;  // ceil(2^32 / F), ceil(2^32 / P): e / F = (e * f_magic) >> 32 for small e
  // lpv_mimo_kernel: the state before every step [B, T, M] as well
  // (nullable; P + M <= kMimoMaxIO planes), m_magic = ceil(2^32 / M)
  E *hs;
  uint64_t m_magic;
  const E *zi;  // [B, M]; nullptr: zeros
  const E *x;   // [B, T, F]
  E *y;         // [B, T, P]
  E *zf;        // [B, M]; nullable (the state after the last step scanned)
  int64_t B, T_len, tiles_per_row;
  uint64_t b_magic;  // tile id -> row by multiply and shift (row_split)
  unsigned b_shift;
  unsigned long long *claims;
  unsigned tiles, per_stripe, spin_limit;
  unsigned agg_only;  // testing: tiles after a row's first publish no inclusive state
  uint64_t *status;
};

// 3 data waves and a look-back wave; a lane owns K consecutive steps (32
// bytes of one feature), a wave 64 K steps.  LDS per data wave: kMimoMaxIO
// planes of 64 K elements, each padded by 16 bytes so that the lanes of a
// staging instruction, which write consecutive elements of different
// planes, spread over the banks.  The outputs overwrite the inputs in the
// same planes: a lane writes step k's outputs after reading its inputs, and
// no other lane reads them.  With separate output planes (60 KB of LDS per
// workgroup at order 4) and 200 VGPRs a CU held two workgroups; at 35 KB and
// 168 VGPRs it holds three.
template <class Alg>
struct MimoShape {
  using E = typename Alg::elem;
  static constexpr int kWaves = 3;
  static constexpr int kThreads = 64 * (kWaves + 1);
  static constexpr int K = 32 / int(sizeof(E));
  static constexpr int kSpan = 64 * K;
  static constexpr int kTile = kWaves * kSpan;
  static constexpr int kPlane = kSpan + 16 / int(sizeof(E));
  static constexpr int kWaveElems = kMimoMaxIO * kPlane;
  // waves per SIMD of the launch bounds: 3 (168 VGPRs), but 2 for order-4
  // fp64, which spilled 14 VGPRs at 168
  static constexpr int kMinWaves = sizeof(E) == 8 && sizeof(typename Alg::s_state) == 4 * sizeof(E) ? 2 : 3;
};

// The model of row b in two halves, each loaded where it is first needed
// (a half that lives across the wave scan holds registers the scan's maps
// want): the input side, A and the columns of B as state vectors; the output
// side, the rows of C as state vectors and D by element.  Zero past F and P,
// so that every step runs the same arithmetic whatever the widths.
template <class Alg>
struct MimoIn {
  typename Alg::s_coef A;
  typename Alg::s_state b[kMimoMaxIO];
};
template <class Alg>
struct MimoOut {
  using E = typename Alg::elem;
  typename Alg::s_state c[kMimoMaxIO];
  E d[kMimoMaxIO][kMimoMaxIO];
};

template <class Alg>
__device__ __forceinline__ MimoIn<Alg> mimo_in(const MimoArgs<Alg> &a, int64_t row) {
  using E = typename Alg::elem;
  using V = SsView<Alg>;
  constexpr int M = V::M;
  MimoIn<Alg> m;
  m.A = V::load_mat(a.A + row * a.A_stride);
  const E *bp = a.Bm + row * a.b_stride;
#pragma unroll
  for (int j = 0; j < kMimoMaxIO; ++j) {
    union {
      typename Alg::s_state s;
      E e[M];
    } u;
#pragma unroll
    for (int i = 0; i < M; ++i) u.e[i] = j < a.F ? bp[i * a.F + j] : E(0);
    m.b[j] = u.s;
  }
  return m;
}

template <class Alg>
__device__ __forceinline__ MimoOut<Alg> mimo_out(const MimoArgs<Alg> &a, int64_t row) {
  using E = typename Alg::elem;
  using V = SsView<Alg>;
  constexpr int M = V::M;
  MimoOut<Alg> m;
  const E *cp = a.Cm + row * a.c_stride;
  const E *dp = a.Dm ? a.Dm + row * a.d_stride : nullptr;
#pragma unroll
  for (int j = 0; j < kMimoMaxIO; ++j) {
    union {
      typename Alg::s_state s;
      E e[M];
    } u;
#pragma unroll
    for (int i = 0; i < M; ++i) u.e[i] = j < a.P ? cp[j * M + i] : E(0);
    m.c[j] = u.s;
#pragma unroll
    for (int f = 0; f < kMimoMaxIO; ++f) m.d[j][f] = (dp && j < a.P && f < a.F) ? dp[j * a.F + f] : E(0);
  }
  return m;
}

// B u for one step's inputs u (zero past F)
template <class Alg>
__device__ __forceinline__ typename Alg::s_state mimo_bx(const MimoIn<Alg> &m, const typename Alg::elem (&u)[kMimoMaxIO]) {
  using E = typename Alg::elem;
  constexpr int M = SsView<Alg>::M;
  union {
    typename Alg::s_state s;
    E e[M];
  } o, ub;
#pragma unroll
  for (int i = 0; i < M; ++i) o.e[i] = E(0);
#pragma unroll
  for (int f = 0; f < kMimoMaxIO; ++f) {
    ub.s = m.b[f];
#pragma unroll
    for (int i = 0; i < M; ++i) o.e[i] = fma(ub.e[i], u[f], o.e[i]);
  }
  return o.s;
}

// A lane's K steps from a zero state, sum_k A^(K-1-k) B x[k], in compute
// precision (the vector part of its map; the matrix part is A^K).  Folding
// in storage precision let float32 rounding in the lane maps of a model
// with a large transient gain reach 3e-4 of the output's range, ten times a
// sequential float32 loop's error; from an exact entry state, pass 2's K
// float32 steps add only a few ulps.
template <class Alg, int K>
__device__ __forceinline__ typename Alg::state mimo_lane_fold(const typename Alg::coef &A,
                                                              const typename Alg::s_state (&X)[K]) {
  typename Alg::state v = Alg::load_s(X[0]);
#pragma unroll
  for (int k = 1; k < K; ++k) v = Alg::affine(A, v, Alg::load_s(X[k]));
  return v;
}

// The elements [lo, hi) of a block of `len` elements starting at element
// `base` of a row of `lim` elements that lie inside the row (clamped to
// [0, len]; lo >= hi when none do).  One bounds test per element serves
// every span: a separate unchecked path for whole spans made the compiler
// keep both paths' loads live (2.9 KB of scratch per lane).
__device__ __forceinline__ void mimo_block_range(int64_t base, int64_t lim, int len, int &lo, int &hi) {
  const int64_t l = base < 0 ? -base : 0, h = lim - base;
  lo = int(l < len ? l : len);
  hi = int(h < 0 ? 0 : (h < len ? h : len));
}

// Stages a wave's span of one [T, W] row block into W LDS planes: plane j
// holds feature j of the span's 64 K steps in scan order (forward: scan
// position s0 + s is time s0 + s; REV: time T-1-s0-s).  Steps outside the
// row read 0.  The global side is the span's contiguous block of 64 K W
// elements, lane-strided (element e = i 64 + lane is step e / W, feature
// e % W of the block).
template <class Alg, bool REV, class Sh = MimoShape<Alg>>
__device__ __forceinline__ void mimo_stage_in(const typename Alg::elem *row, int64_t s0, int64_t T, int W,
                                              uint64_t w_magic, typename Alg::elem *lds, int lane) {
  using E = typename Alg::elem;
  constexpr int S = Sh::kSpan, K = Sh::K, kMax = K * kMimoMaxIO;
  // the block starts at element `base` of the row (negative or past the row
  // for the spans that leave it); its elements [lo, hi) lie inside the row
  const int64_t base = (REV ? T - s0 - S : s0) * W;
  const int n = K * W;  // elements per lane
  int lo, hi;
  mimo_block_range(base, T * W, S * W, lo, hi);
  E v[kMax];
#pragma unroll
  for (int i = 0; i < kMax; ++i) {
    const int e = i * 64 + lane;
    v[i] = E(0);
    if (i < n && e >= lo && e < hi) v[i] = row[base + e];
  }
#pragma unroll
  for (int i = 0; i < kMax; ++i) {
    if (i < n) {
      const unsigned e = unsigned(i * 64 + lane);
      const unsigned s = unsigned((uint64_t(e) * w_magic) >> 32);
      const unsigned j = e - s * unsigned(W);
      lds[j * Sh::kPlane + (REV ? S - 1 - int(s) : int(s))] = v[i];
    }
  }
}

// The inverse of mimo_stage_in for a wave's outputs: W planes out to the
// span's block of the [T, W] row; steps outside the row are not written.
template <class Alg, bool REV, class Sh = MimoShape<Alg>>
__device__ __forceinline__ void mimo_stage_out(typename Alg::elem *row, int64_t s0, int64_t T, int W,
                                               uint64_t w_magic, const typename Alg::elem *lds, int lane) {
  using E = typename Alg::elem;
  constexpr int S = Sh::kSpan, K = Sh::K, kMax = K * kMimoMaxIO;
  const int64_t base = (REV ? T - s0 - S : s0) * W;
  const int n = K * W;
  int lo, hi;
  mimo_block_range(base, T * W, S * W, lo, hi);
  E v[kMax];
#pragma unroll
  for (int i = 0; i < kMax; ++i) {
    if (i < n) {
      const unsigned e = unsigned(i * 64 + lane);
      const unsigned s = unsigned((uint64_t(e) * w_magic) >> 32);
      const unsigned j = e - s * unsigned(W);
      v[i] = lds[j * Sh::kPlane + (REV ? S - 1 - int(s) : int(s))];
    }
  }
#pragma unroll
  for (int i = 0; i < kMax; ++i) {
    const int e = i * 64 + lane;
    if (i < n && e >= lo && e < hi) row[base + e] = v[i];
  }
}

// Time of scan position s in a row of T steps.
template <bool REV>
__device__ __forceinline__ int64_t mimo_time(int64_t s, int64_t T) {
  return REV ? T - 1 - s : s;
}

// State entering tile position `span` of a row, folded from the inputs (the
// look-back's bounded-wait fallback; out of line, cold): 64 K steps at a
// time, each lane reading its K steps' features straight from the row,
// st <- A^(64 K) st + the chunk's total.
template <class Alg, bool REV>
__device__ __noinline__ typename Alg::state mimo_prefix_fallback(const MimoArgs<Alg> *ap, int64_t b, int64_t span,
                                                                int lane, typename Alg::state st,
                                                                const SsPowers<Alg> *tab) {
  const MimoArgs<Alg> &a = *ap;
  using E = typename Alg::elem;
  using SS = typename Alg::s_state;
  constexpr int K = MimoShape<Alg>::K;
  const MimoIn<Alg> mdl = mimo_in<Alg>(a, b);
  const E *xrow = a.x + b * a.T_len * a.F;
  for (int64_t off = 0; off < span; off += 64 * K) {
    ss_reload_tables();
    SS xs[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int64_t s = off + int64_t(lane) * K + k;
      E u[kMimoMaxIO];
#pragma unroll
      for (int f = 0; f < kMimoMaxIO; ++f) {
        u[f] = E(0);
        if (f < a.F && s < a.T_len) u[f] = xrow[mimo_time<REV>(s, a.T_len) * a.F + f];
      }
      xs[k] = mimo_bx<Alg>(mdl, u);
    }
    typename Alg::state v[1] = {mimo_lane_fold<Alg, K>(Alg::load_c(mdl.A), xs)};
    ss_lane_scan<Alg, 1, false>(v, lane, tab->pw);
    st = Alg::affine(tab->pw[6], st, read_lane(v[0], 63));
  }
  return st;
}

template <class Alg, bool REV>
__global__ __launch_bounds__(MimoShape<Alg>::kThreads, MimoShape<Alg>::kMinWaves) void mimo_ss_kernel(MimoArgs<Alg> a) {
  using E = typename Alg::elem;
  using S = typename Alg::state;
  using SS = typename Alg::s_state;
  using V = SsView<Alg>;
  using Sh = MimoShape<Alg>;
  using St = SsStatus<Alg>;
  constexpr int K = Sh::K, kWaves = Sh::kWaves, kP = Sh::kPlane;

  __shared__ S s_wagg[kWaves];  // wave aggregates (matrix part A^(64 K))
  __shared__ S s_wpre[kWaves];  // exclusive wave prefixes (matrix part A^(64 K w))
  __shared__ S s_in;
  __shared__ unsigned s_id, s_tag;
  __shared__ uint64_t s_look[St::kLookWords];
  __shared__ SsPowers<Alg> s_tab;
  __shared__ E s_io[kWaves * Sh::kWaveElems];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the tile is the workgroup's index; the look-back wave claims for the
  // call's tag (claim_tag), so the data waves' loads do not wait for it
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
      const typename Alg::s_coef Arow = V::load_mat(a.A + b * a.A_stride);
      typename Alg::coef P = ss_pow2<Alg>(Arow, __builtin_ctz(K));
#pragma unroll
      for (int i = 0; i < 6; ++i) {
        if (lane == 0) s_tab.pw[i] = P;
        P = Alg::cmul(P, P);
      }
      if (lane == 0) s_tab.pw[6] = P;  // A^(64 K), a wave's span
      if (lane == 0) s_tab.pw[7] = P;
      typename Alg::coef G = P;  // A^(kWaves 64 K), a tile
#pragma unroll
      for (int j = 1; j < kWaves; ++j) G = Alg::cmul(P, G);
#pragma unroll
      for (int j = 0; j < 7; ++j) {
        if (lane == 0) s_tab.gp[j] = G;
        G = Alg::cmul(G, G);
      }
    }
    __syncthreads();  // power tables
    tag = claim_tag(a.claims, a.per_stripe, lane);
    uint64_t *row_status = a.status + b * a.tiles_per_row * St::kStride;
    const S virt = a.zi ? Alg::load_s(V::load_vec(a.zi + b * V::M)) : Alg::szero();
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
        yin = mimo_prefix_fallback<Alg, REV>(kernel_args<MimoArgs<Alg>>(), b, q * Sh::kTile, lane, virt, &s_tab);
    }
    if (q + 1 < a.tiles_per_row && lane == 0 && !(a.agg_only && q > 0))
      publish(row_status + q * St::kStride, Alg::affine(s_tab.gp[0], yin, tagg), tag);
    if (lane == 0) s_in = yin;
    __syncthreads();  // entry state is in s_in
    return;
  }

  // ================= data waves
  E *xin = s_io + w * Sh::kWaveElems;  // F input planes, then P output planes
  E *yout = xin;
  const int64_t s0 = q * Sh::kTile + int64_t(w) * Sh::kSpan;  // the wave's first scan position
  mimo_stage_in<Alg, REV>(a.x + b * T * a.F, s0, T, a.F, a.f_magic, xin, lane);
  const MimoIn<Alg> mi = mimo_in<Alg>(a, b);
  wave_sync();  // the span's inputs are in the planes

  // one step's inputs from the planes (zero past F)
  auto inputs = [&](int k, E (&u)[kMimoMaxIO]) {
#pragma unroll
    for (int f = 0; f < kMimoMaxIO; ++f) u[f] = f < a.F ? xin[f * kP + lane * K + k] : E(0);
  };

  // ---- pass 1: the lane's K steps of B x[t] folded from a zero state, then
  // the wave's vector scan.  Steps past the row's end carry a zero input and
  // only touch the aggregate of its last tile, which nobody reads.
  S v[1];
  {
    SS X[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      E u[kMimoMaxIO];
      inputs(k, u);
      X[k] = mimo_bx<Alg>(mi, u);
    }
    v[0] = mimo_lane_fold<Alg, K>(Alg::load_c(mi.A), X);
  }
  __syncthreads();  // power tables
  ss_lane_scan<Alg, 1, false>(v, lane, s_tab.pw);
  const S prev = shfl_from(v[0], lane - 1);
  S ent[1] = {lane > 0 ? prev : Alg::szero()};
  if (lane == 63) s_wagg[w] = v[0];
  __syncthreads();  // wave aggregates are in s_wagg
  __syncthreads();  // entry state is in s_in
  // the wave's entry state A^(64 K w) s_in + its exclusive prefix; a lane
  // enters at A^(K lane) of that plus its own exclusive prefix
  {
    S st = s_in;
    for (int j = 0; j < w; ++j) st = Alg::affine(s_tab.pw[6], st, Alg::szero());
    st = Alg::sadd(st, s_wpre[w]);
    S sv[1] = {st};
    ss_pow_apply<Alg, 6, 1>(s_tab.pw, lane, sv);
    ent[0] = Alg::sadd(sv[0], ent[0]);
  }
  SS h = Alg::store_s(ent[0]);

  // ---- pass 2: y = C h + D x, then the step (B x again from the planes:
  // keeping the K products from pass 1 held their registers across the scan)
  const MimoOut<Alg> mo = mimo_out<Alg>(a, b);
  const int64_t l0 = s0 + int64_t(lane) * K;  // the lane's first scan position
  const bool has_d = a.Dm != nullptr;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    E u[kMimoMaxIO];
    inputs(k, u);
#pragma unroll
    for (int p = 0; p < kMimoMaxIO; ++p) {
      if (p < a.P) {
        E o = V::dot(mo.c[p], h);
        if (has_d) {
#pragma unroll
          for (int f = 0; f < kMimoMaxIO; ++f) o = fma(mo.d[p][f], u[f], o);
        }
        yout[p * kP + lane * K + k] = o;
      }
    }
    h = Alg::s_affine(mi.A, h, mimo_bx<Alg>(mi, u));
    if (a.zf && l0 + k == T - 1) {
      union {
        SS s;
        E e[V::M];
      } zu;
      zu.s = h;
#pragma unroll
      for (int i = 0; i < V::M; ++i) a.zf[b * V::M + i] = zu.e[i];
    }
  }
  wave_sync();  // the span's outputs are in the planes
  mimo_stage_out<Alg, REV>(a.y + b * T * a.P, s0, T, a.P, a.p_magic, yout, lane);
}

// ---------------------------------------------------------------- time-varying A
// The LPV (parameter-varying) model with several inputs and outputs
// (philtorch/lpv/ssm.py:337-581 with a 3D x or matrix-valued B, C, D that
// are constant in time):
//     h[0] = zi,  y[t] = C h[t] + D x[t],  h[t+1] = A[t] h[t] + B x[t],  zf = h[T]
// A is [rows, T, M, M]; B, C, D and the staging of x and y are the LTI
// kernel's.  Every step has its own matrix, so the scan is the generic
// time-varying one (phs_scan.hpp), as in lpv_ss_kernel: a lane folds its K
// steps (A[t], B x[t]) into a map, wave scans of maps chain the lanes, and
// the look-back resolves map status words.  K is 32 bytes of state-order-2
// coefficients' worth (fp32 8, fp64 4 steps; orders 3-4 half that: a lane
// holds its K matrices).
template <class Alg>
struct LpvMimoShape {
  using E = typename Alg::elem;
  static constexpr int kM = SsView<Alg>::M;
  static constexpr int kWaves = 3;
  static constexpr int kThreads = 64 * (kWaves + 1);
  static constexpr int K = (kM <= 2 ? 32 : 16) / int(sizeof(E));
  static constexpr int kSpan = 64 * K;
  static constexpr int kTile = kWaves * kSpan;
  static constexpr int kPlane = kSpan + 16 / int(sizeof(E));
  static constexpr int kWaveElems = kMimoMaxIO * kPlane;
  // waves per SIMD of the launch bounds: orders 1-2 fit 168 VGPRs (3 waves,
  // three workgroups per CU), orders 3-4 take 256 (2)
  static constexpr int kMinWaves = kM <= 2 ? 3 : 2;
};

// A lane's K matrices A[t] in scan order from scan position s0 (past the
// row: zero), transposed where the adjoint reads them so.
template <class Alg, bool REV, int K>
__device__ __forceinline__ void lpv_mimo_load_A(const MimoArgs<Alg> &a, int64_t b, int64_t s0,
                                                typename Alg::s_coef (&Ak)[K]) {
  using SC = typename Alg::s_coef;
  const SC *row = reinterpret_cast<const SC *>(a.A + b * a.A_stride);
  lpv_load<REV, SC, K>(row, s0, a.T_len, a.A_vec != 0, Ak, Alg::s_czero());
  if (a.A_trans) {
#pragma unroll
    for (int k = 0; k < K; ++k) Ak[k] = Alg::s_adjoint(Ak[k]);  // real: the transpose
  }
}

// State entering tile position `span` of a row, folded from the inputs (the
// look-back's bounded-wait fallback; out of line, cold).
template <class Alg, bool REV>
__device__ __noinline__ typename Alg::state lpv_mimo_prefix_fallback(const MimoArgs<Alg> *ap, int64_t b,
                                                                    int64_t span, int lane,
                                                                    typename Alg::state virt) {
  const MimoArgs<Alg> &a = *ap;
  using E = typename Alg::elem;
  using SC = typename Alg::s_coef;
  using SS = typename Alg::s_state;
  using M = Map<Alg>;
  constexpr int K = LpvMimoShape<Alg>::K;
  auto op = [](const M &p, const M &q) { return compose<Alg>(p, q); };
  const MimoIn<Alg> mdl = mimo_in<Alg>(a, b);  // (its A is not read)
  const E *xrow = a.x + b * a.T_len * a.F;
  const SC dummy = Alg::s_czero();
  M acc = map_identity<Alg>();
  for (int64_t off = 0; off < span; off += 64 * K) {
    const int64_t c0 = off + int64_t(lane) * K;
    SC Ak[K];
    lpv_mimo_load_A<Alg, REV, K>(a, b, c0, Ak);
    SS xs[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int64_t s = c0 + k;
      E u[kMimoMaxIO];
#pragma unroll
      for (int f = 0; f < kMimoMaxIO; ++f) {
        u[f] = E(0);
        if (f < a.F && s < a.T_len) u[f] = xrow[mimo_time<REV>(s, a.T_len) * a.F + f];
      }
      xs[k] = mimo_bx<Alg>(mdl, u);
    }
    M m = lane_map<Alg, true, false, K>(Ak, xs, dummy);
    m = wave_scan_incl(m, lane, op);
    acc = compose<Alg>(acc, read_lane(m, 63));
  }
  return apply<Alg>(acc, virt);
}

// HS: also the state before every step into a.hs (a separate instance, so
// the plain forward carries none of it).
template <class Alg, bool REV, bool HS = false>
__global__ __launch_bounds__(LpvMimoShape<Alg>::kThreads, LpvMimoShape<Alg>::kMinWaves) void lpv_mimo_kernel(
    MimoArgs<Alg> a) {
  using E = typename Alg::elem;
  using S = typename Alg::state;
  using SC = typename Alg::s_coef;
  using SS = typename Alg::s_state;
  using M = Map<Alg>;
  using V = SsView<Alg>;
  using Sh = LpvMimoShape<Alg>;
  using St = StatusShape<Alg>;
  constexpr int K = Sh::K, kWaves = Sh::kWaves, kP = Sh::kPlane;

  __shared__ M s_wagg[kWaves];
  __shared__ M s_wpre[kWaves];
  __shared__ S s_in;
  __shared__ unsigned s_id, s_tag;
  __shared__ uint64_t s_look[St::kLookWords];
  __shared__ E s_io[kWaves * Sh::kWaveElems];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t id = blockIdx.x;
  if (id >= a.tiles) {  // padding of the last stripe round: counted, then gone
    if (tid == 0) claim_tile(a.claims, a.per_stripe, s_id, s_tag);
    return;
  }
  unsigned tag = 0;
  int64_t q, b;  // tile position along the row, row
  split_tile(id, a.B, a.b_magic, a.b_shift, q, b);
  const int64_t T = a.T_len;
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
        yin = lpv_mimo_prefix_fallback<Alg, REV>(kernel_args<MimoArgs<Alg>>(), b, q * Sh::kTile, lane, virt);
    }
    if (q + 1 < a.tiles_per_row && lane == 0 && !(a.agg_only && q > 0))
      publish(row_status + q * St::kStride, apply<Alg>(tagg, yin), tag);
    if (lane == 0) s_in = yin;
    __syncthreads();  // entry state is in s_in
    return;
  }

  // ================= data waves
  E *io = s_io + w * Sh::kWaveElems;  // F input planes, then P output planes
  const int64_t s0 = q * Sh::kTile + int64_t(w) * Sh::kSpan;  // the wave's first scan position
  mimo_stage_in<Alg, REV, Sh>(a.x + b * T * a.F, s0, T, a.F, a.f_magic, io, lane);
  SC Ak[K];
  lpv_mimo_load_A<Alg, REV, K>(a, b, s0 + int64_t(lane) * K, Ak);
  const MimoIn<Alg> mi = mimo_in<Alg>(a, b);  // (its A is not read)
  wave_sync();  // the span's inputs are in the planes

  auto inputs = [&](int k, E (&u)[kMimoMaxIO]) {
#pragma unroll
    for (int f = 0; f < kMimoMaxIO; ++f) u[f] = f < a.F ? io[f * kP + lane * K + k] : E(0);
  };

  // ---- pass 1: the lane map of (A[t], B x[t]) over its K steps, the wave
  // scan.  Steps past the row's end carry a zero matrix and input and only
  // touch the aggregate of its last tile, which nobody reads.
  SS X[K];  // B x[t], kept for pass 2
#pragma unroll
  for (int k = 0; k < K; ++k) {
    E u[kMimoMaxIO];
    inputs(k, u);
    X[k] = mimo_bx<Alg>(mi, u);
  }
  const SC dummy = Alg::s_czero();
  M m = lane_map<Alg, true, false, K>(Ak, X, dummy);
  m = wave_scan_incl(m, lane, op);
  const M ex = wave_shift_up(m, lane, map_identity<Alg>());
  if (lane == 63) s_wagg[w] = m;
  __syncthreads();  // wave aggregates are in s_wagg
  __syncthreads();  // entry state is in s_in
  SS h = Alg::store_s(apply<Alg>(ex, apply<Alg>(s_wpre[w], s_in)));

  // ---- pass 2: y = C h + D x, then the step
  const MimoOut<Alg> mo = mimo_out<Alg>(a, b);
  const int64_t l0 = s0 + int64_t(lane) * K;
  const bool has_d = a.Dm != nullptr;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    E u[kMimoMaxIO];
    if (has_d) inputs(k, u);
#pragma unroll
    for (int p = 0; p < kMimoMaxIO; ++p) {
      if (p < a.P) {
        E o = V::dot(mo.c[p], h);
        if (has_d) {
#pragma unroll
          for (int f = 0; f < kMimoMaxIO; ++f) o = fma(mo.d[p][f], u[f], o);
        }
        io[p * kP + lane * K + k] = o;
      }
    }
    if constexpr (HS) {  // the state before the step into planes P.., the lane's own (already read) slots
      union {
        SS s;
        E e[V::M];
      } hu;
      hu.s = h;
#pragma unroll
      for (int i = 0; i < V::M; ++i) io[(a.P + i) * kP + lane * K + k] = hu.e[i];
    }
    h = Alg::s_affine(Ak[k], h, X[k]);
    if (a.zf && l0 + k == T - 1) {
      union {
        SS s;
        E e[V::M];
      } zu;
      zu.s = h;
#pragma unroll
      for (int i = 0; i < V::M; ++i) a.zf[b * V::M + i] = zu.e[i];
    }
  }
  wave_sync();  // the span's outputs are in the planes
  mimo_stage_out<Alg, REV, Sh>(a.y + b * T * a.P, s0, T, a.P, a.p_magic, io, lane);
  if constexpr (HS) mimo_stage_out<Alg, REV, Sh>(a.hs + b * T * V::M, s0, T, V::M, a.m_magic, io + a.P * kP, lane);
}

}  // namespace phs
