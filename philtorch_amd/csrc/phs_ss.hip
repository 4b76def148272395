// C ABI of the fused single-input, single-output LTI state space and of the
// zero-phase filter built on it (declared in include/philscan.h): argument
// checks, workspace carving and the launches of ss_kernel on the caller's
// stream (one per pass).  No allocation and no synchronisation.
// Workspace layout: [0, 2048) claim header, then the status words of every
// (row, tile).  The coefficient-gradient backward takes a scratch buffer of
// its own for the per-wave partial sums, the row sums and the forward's
// states [B, T, M] (data must never land on the self-resetting status
// words).
#include <type_traits>

#include "phs_launch.hpp"
#include "phs_ss.hpp"

namespace phs {
namespace {

// The shortest tile of any launch mode (the gradient mode's at orders 3-4):
// the workspace and the grid check cover every launch of a call.
template <class Alg>
constexpr int64_t ss_min_tile() {
  return std::min<int64_t>(SsShape<Alg>::kTile, SsShape<Alg, kSsGrad>::kTile);
}

template <class Alg>
size_t ss_ws_bytes(int64_t B, int64_t T) {
  const int64_t tiles = (T + ss_min_tile<Alg>() - 1) / ss_min_tile<Alg>();
  return align_up(align_up(kHeaderBytes) + size_t(B) * size_t(tiles) * SsStatus<Alg>::kStride * sizeof(uint64_t));
}

// Filter mode of the model (SsArgs::filt_form and friends): none, or
// lfilter(b, a) in companion form.
struct SsFilter {
  const void *b = nullptr, *a = nullptr;
  int nb = 0, na = 0, form = 0;
  bool shared = false;
};

// The launch arguments of one pass over [B, T] in launch mode MODE
// (workspace carved as above); false if the workspace is short.
template <class Alg, int MODE = kSsPlain>
bool ss_args(int64_t B, int64_t T, const SsFilter &f, const void *zi, const void *x, void *y, void *zf,
             void *workspace, size_t ws_bytes, SsArgs<Alg> &a) {
  using E = typename Alg::elem;
  using Sh = SsShape<Alg, MODE>;
  const int64_t tiles_per_row = (T + Sh::kTile - 1) / Sh::kTile;
  if (!workspace || ws_bytes < ss_ws_bytes<Alg>(B, T)) return false;
  char *ws = static_cast<char *>(workspace);
  a.fb = static_cast<const E *>(f.b);
  a.fa = static_cast<const E *>(f.a);
  a.nb = f.nb;
  a.na = f.na;
  a.filt_form = f.form;
  a.f_stride_b = f.shared ? 0 : f.nb;
  a.f_stride_a = f.shared ? 0 : f.na;
  a.zi = static_cast<const E *>(zi);
  a.x = static_cast<const E *>(x);
  a.y = static_cast<E *>(y);
  a.zf = static_cast<E *>(zf);
  a.B = B;
  a.T_len = T;
  a.tiles_per_row = tiles_per_row;
  a.claims = reinterpret_cast<unsigned long long *>(ws);
  a.status = reinterpret_cast<uint64_t *>(ws + align_up(kHeaderBytes));
  a.tiles = unsigned(B * tiles_per_row);
  a.per_stripe = (a.tiles + kStripes - 1) / kStripes;
  const unsigned sl = g_spin_limit.load(std::memory_order_relaxed);
  a.spin_limit = sl ? sl : kDefaultSpinLimit;
  a.agg_only = g_agg_only.load(std::memory_order_relaxed) ? 1u : 0u;
  a.vec_ok = (size_t(T) * sizeof(E)) % 16 == 0 && aligned16(x) && aligned16(y);
  return true;
}

// The tile grid is the launched mode's (modes differ in tile length; the
// workspace's status words cover the shortest tiles).
template <class Alg, bool REV, int MODE = kSsPlain>
int ss_launch(SsArgs<Alg> a, hipStream_t stream) {
  using Sh = SsShape<Alg, MODE>;
  a.tiles_per_row = (a.T_len + Sh::kTile - 1) / Sh::kTile;
  a.tiles = unsigned(a.B * a.tiles_per_row);
  a.per_stripe = (a.tiles + kStripes - 1) / kStripes;
  row_split(a.B, a.b_magic, a.b_shift);
  launch_kernel((ss_kernel<Alg, REV, MODE>), dim3(a.per_stripe * kStripes), dim3(Sh::kThreads), 0, stream, a);
  return hipGetLastError() == hipSuccess ? PHS_OK : PHS_ERR_LAUNCH;
}

// The coefficient-gradient backward's scratch: the per-wave partial sums,
// the row sums and the states.
template <class Alg>
struct SsBwdLayout {
  size_t partials = 0, rowsum = 0, states = 0, total = 0;
};
template <class Alg>
SsBwdLayout<Alg> ss_bwd_layout(int64_t B, int64_t T) {
  using C = typename Wide<typename Alg::elem>::type;
  using Sh = SsShape<Alg, kSsGrad>;  // the partials are the gradient launch's
  const int64_t tiles = (T + Sh::kTile - 1) / Sh::kTile;
  SsBwdLayout<Alg> L;
  L.partials = 0;
  L.rowsum = align_up(L.partials + size_t(B) * size_t(tiles) * Sh::kWaves * SsGrad<Alg>::kN * sizeof(C));
  L.states = align_up(L.rowsum + size_t(B) * SsGrad<Alg>::kN * sizeof(C));
  L.total = align_up(L.states + size_t(B) * size_t(T) * sizeof(typename Alg::s_state));
  return L;
}

bool ss_grid_ok(int64_t B, int64_t T, int64_t kTile) {
  return double(B) * double((T + kTile - 1) / kTile) < 2147483648.0;
}

bool ss_filter_ok(const SsFilter &f, int M) {
  return f.nb >= 1 && f.nb <= M + 1 && f.na >= 1 && f.na <= M && (f.nb - 1 == M || f.na == M);
}

template <class Alg>
int ss_fwd(int64_t B, int64_t T, const void *A, bool A_sh, const void *bv, bool b_sh, const void *cv, bool c_sh,
           int out_idx, const void *d, bool d_sh, const SsFilter &f, const void *zi, const void *x, void *y, void *zf,
           void *workspace, size_t ws_bytes, bool rev, hipStream_t stream, void *hs = nullptr) {
  using E = typename Alg::elem;
  constexpr int M = SsView<Alg>::M;
  if (B < 0 || T < 0) return PHS_ERR_INVALID;
  if (f.form == 0 && !cv && (out_idx < 0 || out_idx >= M)) return PHS_ERR_INVALID;
  if (f.form != 0 && !ss_filter_ok(f, M)) return PHS_ERR_INVALID;
  if (B == 0 || T == 0) return PHS_OK;
  if ((f.form == 0 ? !A : (!f.b || !f.a)) || !x || !y) return PHS_ERR_INVALID;
  if (!ss_grid_ok(B, T, SsShape<Alg>::kTile)) return PHS_ERR_INVALID;
  SsArgs<Alg> a{};
  if (!ss_args<Alg>(B, T, f, zi, x, y, zf, workspace, ws_bytes, a)) return PHS_ERR_WORKSPACE;
  a.A = static_cast<const E *>(A);
  a.A_stride = A_sh ? 0 : M * M;
  a.bv = static_cast<const E *>(bv);
  a.b_stride = b_sh ? 0 : M;
  a.cv = static_cast<const E *>(cv);
  a.c_stride = c_sh ? 0 : M;
  a.d = static_cast<const E *>(d);
  a.d_stride = d_sh ? 0 : 1;
  a.out_idx = out_idx;
  if (hs) {  // the states as well, in the same pass (the states-and-output mode)
    a.hs = static_cast<E *>(hs);
    a.vec_hs = aligned16(hs) && (size_t(T) * sizeof(typename Alg::s_state)) % 16 == 0 && aligned16(x) &&
               (size_t(T) * sizeof(E)) % 16 == 0;
    return rev ? ss_launch<Alg, true, kSsStatesY>(a, stream) : ss_launch<Alg, false, kSsStatesY>(a, stream);
  }
  return rev ? ss_launch<Alg, true>(a, stream) : ss_launch<Alg, false>(a, stream);
}

// The explicit model's operands (SsArgs fields of a model with filt_form 0).
template <typename E>
struct SsModelArgs {
  const void *A = nullptr, *b = nullptr, *c = nullptr, *d = nullptr;
  bool A_sh = false, b_sh = false, c_sh = false, d_sh = false;
  int out_idx = 0;
};

// Gradients of y = model(x) (and zf) w.r.t. x, zi and the coefficients:
// the forward again writing its states (kSsStates; skipped when the forward
// kept them, hs_in), the adjoint model in
// the opposite time direction from grad_zf with the coefficient sums
// (kSsGrad; explicit model: A^T, input vector c, output vector b; filter:
// the other companion form of the same b and a), then the row sums and the
// outputs.  gx, gzi and every coefficient output may be null.
template <class Alg>
int ss_bwd(int64_t B, int64_t T, const SsModelArgs<typename Alg::elem> &mo, const SsFilter &f, const void *zi,
           const void *x, const void *gy, const void *gzf, void *gx, void *gzi, SsGradOut<typename Alg::elem> out,
           void *scratch, size_t scratch_bytes, void *workspace, size_t ws_bytes, bool rev, hipStream_t stream,
           const void *hs_in = nullptr) {
  using E = typename Alg::elem;
  using C = typename Wide<E>::type;
  using SS = typename Alg::s_state;
  constexpr int M = SsView<Alg>::M;
  if (B < 0 || T < 0) return PHS_ERR_INVALID;
  if (f.form == 0 && !mo.c && (mo.out_idx < 0 || mo.out_idx >= M)) return PHS_ERR_INVALID;
  if (f.form != 0 && !ss_filter_ok(f, M)) return PHS_ERR_INVALID;
  if (B == 0) return PHS_OK;
  if ((f.form == 0 ? !mo.A : (!f.b || !f.a)) || (T > 0 && (!x || !gy))) return PHS_ERR_INVALID;
  if (f.form == 0 && ((out.gb && !mo.b) || (out.gc && !mo.c) || (out.gd && !mo.d))) return PHS_ERR_INVALID;
  if (!ss_grid_ok(B, T, ss_min_tile<Alg>())) return PHS_ERR_INVALID;
  const SsBwdLayout<Alg> L = ss_bwd_layout<Alg>(B, T);
  if (!scratch || scratch_bytes < L.total) return PHS_ERR_WORKSPACE;
  if (T > 0 && (!workspace || ws_bytes < ss_ws_bytes<Alg>(B, T))) return PHS_ERR_WORKSPACE;
  char *sc = static_cast<char *>(scratch);
  C *gpart = reinterpret_cast<C *>(sc + L.partials);
  C *rowsum = reinterpret_cast<C *>(sc + L.rowsum);
  E *states = hs_in ? const_cast<E *>(static_cast<const E *>(hs_in)) : reinterpret_cast<E *>(sc + L.states);
  const int64_t tiles = (T + SsShape<Alg, kSsGrad>::kTile - 1) / SsShape<Alg, kSsGrad>::kTile;
  auto set_model = [&](SsArgs<Alg> &a, bool adjoint) {
    a.A = static_cast<const E *>(mo.A);
    a.A_stride = mo.A_sh ? 0 : M * M;
    a.A_trans = adjoint ? 1 : 0;
    a.d = static_cast<const E *>(mo.d);
    a.d_stride = mo.d_sh ? 0 : 1;
    const E *bp = static_cast<const E *>(mo.b), *cp = static_cast<const E *>(mo.c);
    if (!adjoint) {
      a.bv = bp, a.b_stride = mo.b_sh ? 0 : M, a.in_idx = 0;
      a.cv = cp, a.c_stride = mo.c_sh ? 0 : M, a.out_idx = mo.out_idx;
    } else {  // input vector c (or e_out_idx), output vector b (or e_0)
      a.bv = cp, a.b_stride = mo.c_sh ? 0 : M, a.in_idx = mo.out_idx;
      a.cv = bp, a.c_stride = mo.b_sh ? 0 : M, a.out_idx = 0;
    }
  };
  if (T > 0) {
    SsArgs<Alg> p{};
    if (!ss_args<Alg>(B, T, f, zi, x, nullptr, nullptr, workspace, ws_bytes, p)) return PHS_ERR_WORKSPACE;
    set_model(p, false);
    p.hs = states;
    p.vec_hs = aligned16(states) && (size_t(T) * sizeof(SS)) % 16 == 0 && aligned16(x) &&
               (size_t(T) * sizeof(E)) % 16 == 0;
    int rc = PHS_OK;
    if (!hs_in) {
      rc = rev ? ss_launch<Alg, true, kSsStates>(p, stream) : ss_launch<Alg, false, kSsStates>(p, stream);
      if (rc != PHS_OK) return rc;
    }
    SsFilter fa = f;
    if (f.form != 0) fa.form = 3 - f.form;  // TDF-II <-> DF-II: the adjoint of a companion form
    if (!ss_args<Alg, kSsGrad>(B, T, fa, gzf, gy, gx, gzi, workspace, ws_bytes, p)) return PHS_ERR_WORKSPACE;
    set_model(p, true);
    p.hs_fwd = states;
    p.x_fwd = static_cast<const E *>(x);
    p.gpart = gpart;
    p.vec_hs = aligned16(states) && (size_t(T) * sizeof(SS)) % 16 == 0 && aligned16(x) &&
               (size_t(T) * sizeof(E)) % 16 == 0;
    rc = rev ? ss_launch<Alg, false, kSsGrad>(p, stream) : ss_launch<Alg, true, kSsGrad>(p, stream);
    if (rc != PHS_OK) return rc;
  }
  out.fb = static_cast<const E *>(f.b);
  out.fa = static_cast<const E *>(f.a);
  out.nb = f.nb;
  out.na = f.na;
  out.form = f.form;
  out.f_sh = f.shared;
  out.gzi = T == 0 ? static_cast<E *>(gzi) : nullptr;
  out.gzf = static_cast<const E *>(gzf);
  hipLaunchKernelGGL(ss_grad_rows_kernel<Alg>, dim3(unsigned(B)), dim3(kSsReduceThreads), 0, stream,
                     static_cast<const C *>(gpart), tiles * SsShape<Alg, kSsGrad>::kWaves, rowsum);
  hipLaunchKernelGGL(ss_grad_finish_kernel<Alg>, dim3(1), dim3(kSsReduceThreads), 0, stream,
                     static_cast<const C *>(rowsum), B, T, out);
  return hipGetLastError() == hipSuccess ? PHS_OK : PHS_ERR_LAUNCH;
}

// filtfilt's scratch buffer ("mid"): pass 1's output [B, T] and final state
// [B, 4] (order 4 at most).  Kept out of the self-resetting workspace, whose
// status words must never be overwritten with data.
inline size_t filtfilt_zf_offset(size_t esz, int64_t B, int64_t T) { return align_up(size_t(B) * size_t(T) * esz); }
inline size_t filtfilt_mid_bytes(size_t esz, int64_t B, int64_t T) {
  return filtfilt_zf_offset(esz, B, T) + align_up(size_t(B) * 4 * esz);
}

// The workspace of either pass at any order (the tile length is the same
// for every order of a precision; the status entries grow with it).
template <typename E>
size_t filtfilt_ws_bytes(int64_t B, int64_t T) {
  size_t m = ss_ws_bytes<Scalar<E>>(B, T);
  m = std::max(m, ss_ws_bytes<Block2<E>>(B, T));
  m = std::max(m, ss_ws_bytes<BlockN<E, 3>>(B, T));
  return std::max(m, ss_ws_bytes<BlockN<E, 4>>(B, T));
}

// Zero-phase filter: pass 1 forward over x from the edge-derived state into
// mid (output and final state), pass 2 in reversed time over mid into y.
// With h1 and h2: both passes also write their states [B, T, M] (the
// states-and-output mode, as the coefficient backward computes them again).
template <class Alg>
int ss_filtfilt(int64_t B, int64_t T, const SsFilter &f, int mode, int64_t e, const void *x, void *y, void *mid,
                void *workspace, size_t ws_bytes, hipStream_t stream, void *h1 = nullptr, void *h2 = nullptr) {
  using E = typename Alg::elem;
  using SS = typename Alg::s_state;
  const bool keep = h1 && h2;
  auto vec_states = [&](const void *hs, const void *xf) {
    return aligned16(hs) && (size_t(T) * sizeof(SS)) % 16 == 0 && aligned16(xf) && (size_t(T) * sizeof(E)) % 16 == 0;
  };
  if (ws_bytes < filtfilt_ws_bytes<E>(B, T)) return PHS_ERR_WORKSPACE;  // the documented size, any order
  char *m = static_cast<char *>(mid);
  E *y1 = reinterpret_cast<E *>(m);
  E *zf1 = reinterpret_cast<E *>(m + filtfilt_zf_offset(sizeof(E), B, T));
  SsArgs<Alg> p{};
  if (!ss_args<Alg>(B, T, f, nullptr, x, y1, zf1, workspace, ws_bytes, p)) return PHS_ERR_WORKSPACE;
  p.virt_mode = 1;
  p.xpad = static_cast<const E *>(x);
  p.pad_mode = mode;
  p.pad_len = e;
  if (keep) {
    p.hs = static_cast<E *>(h1);
    p.vec_hs = vec_states(h1, x);
  }
  int rc = keep ? ss_launch<Alg, false, kSsStatesY>(p, stream) : ss_launch<Alg, false>(p, stream);
  if (rc != PHS_OK) return rc;
  if (!ss_args<Alg>(B, T, f, nullptr, y1, y, nullptr, workspace, ws_bytes, p)) return PHS_ERR_WORKSPACE;
  p.virt_mode = 2;
  p.xpad = static_cast<const E *>(x);
  p.zf_prev = zf1;
  p.pad_mode = mode;
  p.pad_len = e;
  if (keep) {
    p.hs = static_cast<E *>(h2);
    p.vec_hs = vec_states(h2, y1);
    return ss_launch<Alg, true, kSsStatesY>(p, stream);
  }
  return ss_launch<Alg, true>(p, stream);
}

// filtfilt backward's scratch: pass 1's adjoint input dL/dy1 over the
// interior [B, T], the three [B, 4] adjoint states (after pass 2's interior,
// entering and after pass 1's) and the back pad's values [B, padlen] in
// double; with coefficient gradients also pass 1's output and final state,
// both passes' interior states [B, T, M], the per-wave partial sums (one
// buffer, used by each adjoint launch in turn), two [B, kN] row sums, dL/dz
// [B, M] and, for pads longer than kFfPadLds, the pads' working values
// [B, padlen, 2M + 2] in double.
template <class Alg>
struct FfBwdLayout {
  size_t gy1 = 0, lam_a = 0, entry = 0, lam_b = 0, edge = 0;
  size_t y1 = 0, zf1 = 0, h1 = 0, h2 = 0, gpart = 0, rowsum1 = 0, rowsum2 = 0, gz = 0, work = 0, total = 0;
};
template <class Alg>
FfBwdLayout<Alg> ff_bwd_layout(int64_t B, int64_t T, int64_t e, bool coef) {
  using E = typename Alg::elem;
  using C = typename Wide<E>::type;
  constexpr int M = SsView<Alg>::M;
  const size_t esz = sizeof(E), rows = size_t(B), n = size_t(B) * size_t(T);
  FfBwdLayout<Alg> L;
  L.lam_a = align_up(n * esz);
  L.entry = L.lam_a + align_up(rows * 4 * esz);
  L.lam_b = L.entry + align_up(rows * 4 * esz);
  L.edge = L.lam_b + align_up(rows * 4 * esz);
  L.total = L.edge + align_up(rows * size_t(e) * sizeof(double));
  if (!coef) return L;
  const int64_t tiles = (T + SsShape<Alg, kSsGrad>::kTile - 1) / SsShape<Alg, kSsGrad>::kTile;
  constexpr int N = SsGrad<Alg>::kN;
  L.y1 = L.total;
  L.zf1 = L.y1 + align_up(n * esz);
  L.h1 = L.zf1 + align_up(rows * M * esz);
  L.h2 = L.h1 + align_up(n * sizeof(typename Alg::s_state));
  L.gpart = L.h2 + align_up(n * sizeof(typename Alg::s_state));
  L.rowsum1 = L.gpart + align_up(rows * size_t(tiles) * SsShape<Alg, kSsGrad>::kWaves * N * sizeof(C));
  L.rowsum2 = L.rowsum1 + align_up(rows * N * sizeof(C));
  L.gz = L.rowsum2 + align_up(rows * N * sizeof(C));
  L.work = L.gz + align_up(rows * M * sizeof(double));
  L.total = L.work + align_up(rows * size_t(e > kFfPadLds ? e : 0) * FfPad<M>::kW * sizeof(double));
  return L;
}

// Gradients of the zero-phase filter (ff_bwd_edge_kernel's comment).  Input
// only: pass 2's adjoint over the interior, the back pad (edge kernel),
// pass 1's adjoint over the interior in reversed time, the front pad and
// the fold (fold kernel).  Both adjoint launches run the DF-II form of the
// same b and a, the adjoint of the TDF-II model the forward runs.  With
// coefficient gradients (gfb, gfa) first pass 1 again keeping its states,
// output and final state (kSsStatesY) and pass 2 keeping its states
// (kSsStates), then the adjoint launches in the gradient mode, each
// followed by its row sums, the pads' sums and dL/dz in the edge and fold
// kernels, and the filter chain rule (ss_grad_finish_kernel).
template <class Alg>
int ss_filtfilt_bwd(int64_t B, int64_t T, const SsFilter &f, int mode, int64_t e, const void *x, const void *gy,
                    void *gx, void *gfb, void *gfa, void *scratch, size_t scratch_bytes, void *workspace,
                    size_t ws_bytes, hipStream_t stream, const void *mid_in = nullptr, const void *h1_in = nullptr,
                    const void *h2_in = nullptr) {
  using E = typename Alg::elem;
  using C = typename Wide<E>::type;
  using SS = typename Alg::s_state;
  constexpr int M = SsView<Alg>::M;
  static_assert(std::is_same<C, double>::value, "row sums in double");
  static_assert(FfSums<M>::kN == SsGrad<Alg>::kN && FfSums<M>::kB == SsGrad<Alg>::kB &&
                    FfSums<M>::kD == SsGrad<Alg>::kD,
                "the pads' sums in the kernels' layout");
  const bool coef = gfb != nullptr;
  if (!ss_grid_ok(B, T, ss_min_tile<Alg>())) return PHS_ERR_INVALID;
  if (ws_bytes < filtfilt_ws_bytes<E>(B, T)) return PHS_ERR_WORKSPACE;
  const FfBwdLayout<Alg> L = ff_bwd_layout<Alg>(B, T, e, coef);
  if (!scratch || scratch_bytes < L.total) return PHS_ERR_WORKSPACE;
  char *sc = static_cast<char *>(scratch);
  auto at = [&](size_t off) { return static_cast<void *>(sc + off); };
  FfBwdArgs<E> k{};
  k.fb = static_cast<const E *>(f.b);
  k.fa = static_cast<const E *>(f.a);
  k.nb = f.nb;
  k.na = f.na;
  k.f_stride_b = f.shared ? 0 : f.nb;
  k.f_stride_a = f.shared ? 0 : f.na;
  k.B = B;
  k.T = T;
  k.e = e;
  k.pad_mode = mode;
  E *gy1 = static_cast<E *>(at(L.gy1));
  E *lam_a = static_cast<E *>(at(L.lam_a));
  E *entry = static_cast<E *>(at(L.entry));
  E *lam_b = static_cast<E *>(at(L.lam_b));
  k.lam_a = lam_a;
  k.gy1 = gy1;
  k.edge = static_cast<double *>(at(L.edge));
  k.entry = entry;
  k.lam_b = lam_b;
  k.gx = static_cast<E *>(gx);
  const int64_t tiles = (T + SsShape<Alg, kSsGrad>::kTile - 1) / SsShape<Alg, kSsGrad>::kTile;
  const dim3 grid(unsigned((B + kFfRows - 1) / kFfRows));
  const bool lds = e <= kFfPadLds;
  SsFilter adj = f;
  adj.form = 2;
  SsArgs<Alg> p{};
  int rc = PHS_OK;
  E *y1 = nullptr, *zf1 = nullptr;
  SS *h1 = nullptr, *h2 = nullptr;
  C *gpart = nullptr, *rowsum1 = nullptr, *rowsum2 = nullptr;
  auto vec_states = [&](const void *hs, const void *xf) {
    return aligned16(hs) && (size_t(T) * sizeof(SS)) % 16 == 0 && aligned16(xf) && (size_t(T) * sizeof(E)) % 16 == 0;
  };
  if (coef) {
    y1 = static_cast<E *>(at(L.y1));
    zf1 = static_cast<E *>(at(L.zf1));
    h1 = static_cast<SS *>(at(L.h1));
    h2 = static_cast<SS *>(at(L.h2));
    gpart = static_cast<C *>(at(L.gpart));
    rowsum1 = static_cast<C *>(at(L.rowsum1));
    rowsum2 = static_cast<C *>(at(L.rowsum2));
    k.coef = 1;
    k.x = static_cast<const E *>(x);
    k.y1 = y1;
    k.zf1 = zf1;
    k.work = static_cast<double *>(at(L.work));
    k.gz = static_cast<double *>(at(L.gz));
    k.rowsum1 = rowsum1;
    k.rowsum2 = rowsum2;
  }
  if (coef && mid_in && h1_in && h2_in) {
    // the forward kept pass 1's output and final state and both passes' states
    char *m = static_cast<char *>(const_cast<void *>(mid_in));
    y1 = reinterpret_cast<E *>(m);
    zf1 = reinterpret_cast<E *>(m + filtfilt_zf_offset(sizeof(E), B, T));
    h1 = static_cast<SS *>(const_cast<void *>(h1_in));
    h2 = static_cast<SS *>(const_cast<void *>(h2_in));
    k.y1 = y1;
    k.zf1 = zf1;
  } else if (coef) {
    // pass 1 (states, output, final state), then pass 2 (states)
    if (!ss_args<Alg>(B, T, f, nullptr, x, y1, zf1, workspace, ws_bytes, p)) return PHS_ERR_WORKSPACE;
    p.virt_mode = 1;
    p.xpad = static_cast<const E *>(x);
    p.pad_mode = mode;
    p.pad_len = e;
    p.hs = reinterpret_cast<E *>(h1);
    p.vec_hs = vec_states(h1, x);
    if ((rc = ss_launch<Alg, false, kSsStatesY>(p, stream)) != PHS_OK) return rc;
    p = SsArgs<Alg>{};
    if (!ss_args<Alg>(B, T, f, nullptr, y1, nullptr, nullptr, workspace, ws_bytes, p)) return PHS_ERR_WORKSPACE;
    p.virt_mode = 2;
    p.xpad = static_cast<const E *>(x);
    p.zf_prev = zf1;
    p.pad_mode = mode;
    p.pad_len = e;
    p.hs = reinterpret_cast<E *>(h2);
    p.vec_hs = vec_states(h2, y1);
    if ((rc = ss_launch<Alg, true, kSsStates>(p, stream)) != PHS_OK) return rc;
  }
  // pass 2's adjoint over the interior (ascending time)
  p = SsArgs<Alg>{};
  const bool args_ok = coef ? ss_args<Alg, kSsGrad>(B, T, adj, nullptr, gy, gy1, lam_a, workspace, ws_bytes, p)
                             : ss_args<Alg>(B, T, adj, nullptr, gy, gy1, lam_a, workspace, ws_bytes, p);
  if (!args_ok) return PHS_ERR_WORKSPACE;
  if (coef) {
    p.hs_fwd = reinterpret_cast<const E *>(h2);
    p.x_fwd = y1;
    p.gpart = gpart;
    p.vec_hs = vec_states(h2, y1);
    if ((rc = ss_launch<Alg, false, kSsGrad>(p, stream)) != PHS_OK) return rc;
    hipLaunchKernelGGL(ss_grad_rows_kernel<Alg>, dim3(unsigned(B)), dim3(kSsReduceThreads), 0, stream,
                       static_cast<const C *>(gpart), tiles * SsShape<Alg, kSsGrad>::kWaves, rowsum2);
  } else if ((rc = ss_launch<Alg, false>(p, stream)) != PHS_OK) {
    return rc;
  }
  if (lds)
    hipLaunchKernelGGL((ff_bwd_edge_kernel<E, M, kFfPadLds>), grid, dim3(kFfRows), 0, stream, k);
  else
    hipLaunchKernelGGL((ff_bwd_edge_kernel<E, M, 0>), grid, dim3(kFfRows), 0, stream, k);
  // pass 1's adjoint over the interior (descending time)
  p = SsArgs<Alg>{};
  const bool args1_ok = coef ? ss_args<Alg, kSsGrad>(B, T, adj, entry, gy1, gx, lam_b, workspace, ws_bytes, p)
                              : ss_args<Alg>(B, T, adj, entry, gy1, gx, lam_b, workspace, ws_bytes, p);
  if (!args1_ok) return PHS_ERR_WORKSPACE;
  if (coef) {
    p.hs_fwd = reinterpret_cast<const E *>(h1);
    p.x_fwd = static_cast<const E *>(x);
    p.gpart = gpart;
    p.vec_hs = vec_states(h1, x);
    if ((rc = ss_launch<Alg, true, kSsGrad>(p, stream)) != PHS_OK) return rc;
    hipLaunchKernelGGL(ss_grad_rows_kernel<Alg>, dim3(unsigned(B)), dim3(kSsReduceThreads), 0, stream,
                       static_cast<const C *>(gpart), tiles * SsShape<Alg, kSsGrad>::kWaves, rowsum1);
  } else if ((rc = ss_launch<Alg, true>(p, stream)) != PHS_OK) {
    return rc;
  }
  if (lds)
    hipLaunchKernelGGL((ff_bwd_fold_kernel<E, M, kFfPadLds>), grid, dim3(kFfRows), 0, stream, k);
  else
    hipLaunchKernelGGL((ff_bwd_fold_kernel<E, M, 0>), grid, dim3(kFfRows), 0, stream, k);
  if (coef) {
    SsGradOut<E> out{};
    out.form = 1;
    out.f_sh = f.shared;
    out.fb = static_cast<const E *>(f.b);
    out.fa = static_cast<const E *>(f.a);
    out.nb = f.nb;
    out.na = f.na;
    out.gfb = static_cast<E *>(gfb);
    out.gfa = static_cast<E *>(gfa);
    hipLaunchKernelGGL(ss_grad_finish_kernel<Alg>, dim3(1), dim3(kSsReduceThreads), 0, stream,
                       static_cast<const C *>(rowsum1), B, T, out);
  }
  return hipGetLastError() == hipSuccess ? PHS_OK : PHS_ERR_LAUNCH;
}

// f(Alg{}) for one of the eight (dtype, M) models
template <class F>
int ss_dispatch(int dtype, int M, F &&f) {
  if (dtype != PHS_F32 && dtype != PHS_F64) return PHS_ERR_DTYPE;
  const bool f32 = dtype == PHS_F32;
  switch (M) {
    case 1: return f32 ? f(Scalar<float>{}) : f(Scalar<double>{});
    case 2: return f32 ? f(Block2<float>{}) : f(Block2<double>{});
    case 3: return f32 ? f(BlockN<float, 3>{}) : f(BlockN<double, 3>{});
    case 4: return f32 ? f(BlockN<float, 4>{}) : f(BlockN<double, 4>{});
    default: return PHS_ERR_INVALID;
  }
}

}  // namespace

// One biquad, lfilter(b, a, form="tdf2") with b [rows, nb] and a [rows, 2] at
// their own row strides (0 = shared), as the plain state-space pass, writing
// the fused cascade's checkpoints at one section (the state entering every
// ckpt_every-th step, [B, n_ckpt] in compute precision; nullable) for its
// gradient backward (phs_biquad_fwd).
int biquad_fwd_ss(int dtype, int64_t B, int64_t T, const void *b, int nb, int64_t b_row_stride, const void *a,
                  int64_t a_row_stride, const void *zi, const void *x, void *y, void *zf, void *ckpt, int64_t n_ckpt,
                  int ckpt_every, void *workspace, size_t ws_bytes, hipStream_t stream) {
  auto run = [&](auto alg) -> int {
    using Alg = decltype(alg);
    SsFilter f;
    f.b = b, f.a = a, f.nb = nb, f.na = 2, f.form = 1;
    if (B < 0 || T < 0 || b_row_stride < 0 || a_row_stride < 0 || !ss_filter_ok(f, 2)) return PHS_ERR_INVALID;
    if (B == 0 || T == 0) return PHS_OK;
    if (!b || !a || !x || !y || (ckpt && (ckpt_every <= 0 || ckpt_every % SsShape<Alg>::K != 0))) return PHS_ERR_INVALID;
    if (!ss_grid_ok(B, T, SsShape<Alg>::kTile)) return PHS_ERR_INVALID;
    SsArgs<Alg> p{};
    if (!ss_args<Alg>(B, T, f, zi, x, y, zf, workspace, ws_bytes, p)) return PHS_ERR_WORKSPACE;
    p.f_stride_b = b_row_stride;
    p.f_stride_a = a_row_stride;
    p.ckpt = ckpt;
    p.n_ckpt = n_ckpt;
    p.ckpt_every = ckpt_every;
    return ss_launch<Alg, false>(p, stream);
  };
  switch (dtype) {
    case PHS_F32: return run(Block2<float>{});
    case PHS_F64: return run(Block2<double>{});
    default: return PHS_ERR_DTYPE;
  }
}

size_t biquad_ss_ws_bytes(int dtype, int64_t B, int64_t T) {
  if (B <= 0 || T <= 0) return 0;
  switch (dtype) {
    case PHS_F32: return ss_ws_bytes<Block2<float>>(B, T);
    case PHS_F64: return ss_ws_bytes<Block2<double>>(B, T);
    default: return 0;
  }
}

}  // namespace phs

extern "C" {

size_t phs_lti_ss_workspace_size(int dtype, int M, int64_t B, int64_t T) {
  if (B < 0 || T < 0) return 0;
  size_t out = 0;
  const int rc = phs::ss_dispatch(dtype, M, [&](auto alg) {
    out = phs::ss_ws_bytes<decltype(alg)>(B, T);
    return PHS_OK;
  });
  return rc == PHS_OK ? out : 0;
}

namespace {

int lti_ss_call(int dtype, int M, int64_t B, int64_t T, const void *A, int A_shared, const void *b, int b_shared,
                const void *c, int c_shared, int out_idx, const void *d, int d_shared, const void *zi, const void *x,
                void *y, void *zf, void *workspace, size_t workspace_bytes, bool rev, void *stream,
                void *hs = nullptr) {
  const hipStream_t st = static_cast<hipStream_t>(stream);
  return phs::ss_dispatch(dtype, M, [&](auto alg) {
    return phs::ss_fwd<decltype(alg)>(B, T, A, A_shared != 0, b, b_shared != 0, c, c_shared != 0, out_idx, d,
                                      d_shared != 0, phs::SsFilter{}, zi, x, y, zf, workspace, workspace_bytes, rev,
                                      st, hs);
  });
}

int lfilter_call(int dtype, int64_t B, int64_t T, const void *b, int nb, const void *a, int na, int coef_shared,
                 int form, const void *zi, const void *x, void *y, void *zf, void *workspace, size_t workspace_bytes,
                 bool rev, void *stream, void *hs = nullptr) {
  if (form != PHS_FORM_TDF2 && form != PHS_FORM_DF2) return PHS_ERR_INVALID;
  const int M = nb - 1 > na ? nb - 1 : na;
  if (M < 1 || M > 4) return PHS_ERR_INVALID;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  phs::SsFilter f;
  f.b = b;
  f.a = a;
  f.nb = nb;
  f.na = na;
  f.form = form == PHS_FORM_TDF2 ? 1 : 2;
  f.shared = coef_shared != 0;
  return phs::ss_dispatch(dtype, M, [&](auto alg) {
    return phs::ss_fwd<decltype(alg)>(B, T, nullptr, false, nullptr, false, nullptr, false, 0, nullptr, false, f, zi,
                                      x, y, zf, workspace, workspace_bytes, rev, st, hs);
  });
}

}  // namespace

int phs_lti_ss_fwd(int dtype, int M, int64_t B, int64_t T, const void *A, int A_shared, const void *b, int b_shared,
                   const void *c, int c_shared, int out_idx, const void *d, int d_shared, const void *zi,
                   const void *x, void *y, void *zf, void *workspace, size_t workspace_bytes, void *stream) {
  return lti_ss_call(dtype, M, B, T, A, A_shared, b, b_shared, c, c_shared, out_idx, d, d_shared, zi, x, y, zf,
                     workspace, workspace_bytes, false, stream);
}

int phs_lti_ss_rev(int dtype, int M, int64_t B, int64_t T, const void *A, int A_shared, const void *b, int b_shared,
                   const void *c, int c_shared, int out_idx, const void *d, int d_shared, const void *zi,
                   const void *x, void *y, void *zf, void *workspace, size_t workspace_bytes, void *stream) {
  return lti_ss_call(dtype, M, B, T, A, A_shared, b, b_shared, c, c_shared, out_idx, d, d_shared, zi, x, y, zf,
                     workspace, workspace_bytes, true, stream);
}

int phs_lfilter_fwd(int dtype, int64_t B, int64_t T, const void *b, int nb, const void *a, int na, int coef_shared,
                    int form, const void *zi, const void *x, void *y, void *zf, void *workspace,
                    size_t workspace_bytes, void *stream) {
  return lfilter_call(dtype, B, T, b, nb, a, na, coef_shared, form, zi, x, y, zf, workspace, workspace_bytes, false,
                      stream);
}

int phs_lfilter_rev(int dtype, int64_t B, int64_t T, const void *b, int nb, const void *a, int na, int coef_shared,
                    int form, const void *zi, const void *x, void *y, void *zf, void *workspace,
                    size_t workspace_bytes, void *stream) {
  return lfilter_call(dtype, B, T, b, nb, a, na, coef_shared, form, zi, x, y, zf, workspace, workspace_bytes, true,
                      stream);
}

int phs_lti_ss_fwd_hs(int dtype, int M, int64_t B, int64_t T, const void *A, int A_shared, const void *b,
                      int b_shared, const void *c, int c_shared, int out_idx, const void *d, int d_shared,
                      const void *zi, const void *x, void *y, void *zf, void *hs, int reverse, void *workspace,
                      size_t workspace_bytes, void *stream) {
  if (!hs && B > 0 && T > 0) return PHS_ERR_INVALID;
  return lti_ss_call(dtype, M, B, T, A, A_shared, b, b_shared, c, c_shared, out_idx, d, d_shared, zi, x, y, zf,
                     workspace, workspace_bytes, reverse != 0, stream, hs);
}

int phs_lfilter_fwd_hs(int dtype, int64_t B, int64_t T, const void *b, int nb, const void *a, int na,
                       int coef_shared, int form, const void *zi, const void *x, void *y, void *zf, void *hs,
                       int reverse, void *workspace, size_t workspace_bytes, void *stream) {
  if (!hs && B > 0 && T > 0) return PHS_ERR_INVALID;
  return lfilter_call(dtype, B, T, b, nb, a, na, coef_shared, form, zi, x, y, zf, workspace, workspace_bytes,
                      reverse != 0, stream, hs);
}

size_t phs_lti_ss_bwd_scratch_size(int dtype, int M, int64_t B, int64_t T) {
  if (B < 0 || T < 0) return 0;
  size_t out = 0;
  const int rc = phs::ss_dispatch(dtype, M, [&](auto alg) {
    out = phs::ss_bwd_layout<decltype(alg)>(B, T).total;
    return PHS_OK;
  });
  return rc == PHS_OK ? out : 0;
}

int phs_lti_ss_bwd(int dtype, int M, int64_t B, int64_t T, const void *A, int A_shared, const void *b, int b_shared,
                   const void *c, int c_shared, int out_idx, const void *d, int d_shared, const void *zi,
                   const void *x, const void *gy, const void *gzf, void *gx, void *gzi, void *gA, void *gb, void *gc,
                   void *gd, int reverse, void *scratch, size_t scratch_bytes, void *workspace,
                   size_t workspace_bytes, void *stream) {
  return phs_lti_ss_bwd_hs(dtype, M, B, T, A, A_shared, b, b_shared, c, c_shared, out_idx, d, d_shared, zi, x,
                           nullptr, gy, gzf, gx, gzi, gA, gb, gc, gd, reverse, scratch, scratch_bytes, workspace,
                           workspace_bytes, stream);
}

int phs_lti_ss_bwd_hs(int dtype, int M, int64_t B, int64_t T, const void *A, int A_shared, const void *b,
                      int b_shared, const void *c, int c_shared, int out_idx, const void *d, int d_shared,
                      const void *zi, const void *x, const void *hs, const void *gy, const void *gzf, void *gx,
                      void *gzi, void *gA, void *gb, void *gc, void *gd, int reverse, void *scratch,
                      size_t scratch_bytes, void *workspace, size_t workspace_bytes, void *stream) {
  const hipStream_t st = static_cast<hipStream_t>(stream);
  return phs::ss_dispatch(dtype, M, [&](auto alg) {
    using Alg = decltype(alg);
    using E = typename Alg::elem;
    phs::SsModelArgs<E> mo;
    mo.A = A, mo.b = b, mo.c = c, mo.d = d;
    mo.A_sh = A_shared != 0, mo.b_sh = b_shared != 0, mo.c_sh = c_shared != 0, mo.d_sh = d_shared != 0;
    mo.out_idx = out_idx;
    phs::SsGradOut<E> o{};
    o.gA = static_cast<E *>(gA), o.gb = static_cast<E *>(gb), o.gc = static_cast<E *>(gc), o.gd = static_cast<E *>(gd);
    o.A_sh = mo.A_sh, o.b_sh = mo.b_sh, o.c_sh = mo.c_sh, o.d_sh = mo.d_sh;
    return phs::ss_bwd<Alg>(B, T, mo, phs::SsFilter{}, zi, x, gy, gzf, gx, gzi, o, scratch, scratch_bytes, workspace,
                            workspace_bytes, reverse != 0, st, hs);
  });
}

int phs_lfilter_bwd(int dtype, int64_t B, int64_t T, const void *b, int nb, const void *a, int na, int coef_shared,
                    int form, const void *zi, const void *x, const void *gy, const void *gzf, void *gx, void *gzi,
                    void *gb, void *ga, int reverse, void *scratch, size_t scratch_bytes, void *workspace,
                    size_t workspace_bytes, void *stream) {
  return phs_lfilter_bwd_hs(dtype, B, T, b, nb, a, na, coef_shared, form, zi, x, nullptr, gy, gzf, gx, gzi, gb, ga,
                            reverse, scratch, scratch_bytes, workspace, workspace_bytes, stream);
}

int phs_lfilter_bwd_hs(int dtype, int64_t B, int64_t T, const void *b, int nb, const void *a, int na,
                       int coef_shared, int form, const void *zi, const void *x, const void *hs, const void *gy,
                       const void *gzf, void *gx, void *gzi, void *gb, void *ga, int reverse, void *scratch,
                       size_t scratch_bytes, void *workspace, size_t workspace_bytes, void *stream) {
  if (form != PHS_FORM_TDF2 && form != PHS_FORM_DF2) return PHS_ERR_INVALID;
  const int M = nb - 1 > na ? nb - 1 : na;
  if (M < 1 || M > 4 || !gb || !ga) return PHS_ERR_INVALID;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  phs::SsFilter f;
  f.b = b;
  f.a = a;
  f.nb = nb;
  f.na = na;
  f.form = form == PHS_FORM_TDF2 ? 1 : 2;
  f.shared = coef_shared != 0;
  return phs::ss_dispatch(dtype, M, [&](auto alg) {
    using Alg = decltype(alg);
    using E = typename Alg::elem;
    phs::SsGradOut<E> o{};
    o.gfb = static_cast<E *>(gb);
    o.gfa = static_cast<E *>(ga);
    return phs::ss_bwd<Alg>(B, T, phs::SsModelArgs<E>{}, f, zi, x, gy, gzf, gx, gzi, o, scratch, scratch_bytes,
                            workspace, workspace_bytes, reverse != 0, st, hs);
  });
}

size_t phs_filtfilt_workspace_size(int dtype, int64_t B, int64_t T) {
  if (B < 0 || T < 1) return 0;
  switch (dtype) {
    case PHS_F32: return phs::filtfilt_ws_bytes<float>(B, T);
    case PHS_F64: return phs::filtfilt_ws_bytes<double>(B, T);
    default: return 0;
  }
}

size_t phs_filtfilt_mid_size(int dtype, int64_t B, int64_t T) {
  if (B < 0 || T < 1) return 0;
  switch (dtype) {
    case PHS_F32: return phs::filtfilt_mid_bytes(sizeof(float), B, T);
    case PHS_F64: return phs::filtfilt_mid_bytes(sizeof(double), B, T);
    default: return 0;
  }
}

int phs_filtfilt_fwd(int dtype, int64_t B, int64_t T, const void *b, int nb, const void *a, int na,
                     int coef_shared, int padmode, int64_t padlen, const void *x, void *y, void *mid, void *workspace,
                     size_t workspace_bytes, void *stream) {
  return phs_filtfilt_fwd_hs(dtype, B, T, b, nb, a, na, coef_shared, padmode, padlen, x, y, mid, nullptr, nullptr,
                             workspace, workspace_bytes, stream);
}

int phs_filtfilt_fwd_hs(int dtype, int64_t B, int64_t T, const void *b, int nb, const void *a, int na,
                        int coef_shared, int padmode, int64_t padlen, const void *x, void *y, void *mid, void *h1,
                        void *h2, void *workspace, size_t workspace_bytes, void *stream) {
  if (dtype != PHS_F32 && dtype != PHS_F64) return PHS_ERR_DTYPE;
  if ((h1 == nullptr) != (h2 == nullptr)) return PHS_ERR_INVALID;
  const int M = nb - 1 > na ? nb - 1 : na;
  if (B < 0 || T < 1 || nb < 1 || nb > 5 || na < 1 || na > 4 || padlen < 0 || padlen >= T ||
      padmode < PHS_PAD_CONSTANT || padmode > PHS_PAD_CIRCULAR)
    return PHS_ERR_INVALID;
  if (B == 0) return PHS_OK;
  if (!b || !a || !x || !y || !mid) return PHS_ERR_INVALID;
  const int64_t tile = dtype == PHS_F32 ? phs::SsShape<phs::Scalar<float>>::kTile : phs::SsShape<phs::Scalar<double>>::kTile;
  if (!phs::ss_grid_ok(B, T, tile)) return PHS_ERR_INVALID;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  phs::SsFilter f;
  f.b = b;
  f.a = a;
  f.nb = nb;
  f.na = na;
  f.form = 1;  // TDF-II (ss_filtfilt_entry)
  f.shared = coef_shared != 0;
  return phs::ss_dispatch(dtype, M, [&](auto alg) {
    return phs::ss_filtfilt<decltype(alg)>(B, T, f, padmode, padlen, x, y, mid, workspace, workspace_bytes, st, h1,
                                           h2);
  });
}

size_t phs_filtfilt_bwd_scratch_size(int dtype, int M, int64_t B, int64_t T, int64_t padlen, int need_coef) {
  if (B < 0 || T < 0 || padlen < 0 || M < 1 || M > 4) return 0;
  size_t n = 0;
  if (phs::ss_dispatch(dtype, M, [&](auto alg) {
        n = phs::ff_bwd_layout<decltype(alg)>(B, T, padlen, need_coef != 0).total;
        return PHS_OK;
      }) != PHS_OK)
    return 0;
  return n;
}

int phs_filtfilt_bwd(int dtype, int64_t B, int64_t T, const void *b, int nb, const void *a, int na,
                     int coef_shared, int padmode, int64_t padlen, const void *x, const void *grad_y, void *grad_x,
                     void *grad_b, void *grad_a, void *scratch, size_t scratch_bytes, void *workspace,
                     size_t workspace_bytes, void *stream) {
  return phs_filtfilt_bwd_hs(dtype, B, T, b, nb, a, na, coef_shared, padmode, padlen, x, nullptr, nullptr, nullptr,
                             grad_y, grad_x, grad_b, grad_a, scratch, scratch_bytes, workspace, workspace_bytes,
                             stream);
}

int phs_filtfilt_bwd_hs(int dtype, int64_t B, int64_t T, const void *b, int nb, const void *a, int na,
                        int coef_shared, int padmode, int64_t padlen, const void *x, const void *mid, const void *h1,
                        const void *h2, const void *grad_y, void *grad_x, void *grad_b, void *grad_a, void *scratch,
                        size_t scratch_bytes, void *workspace, size_t workspace_bytes, void *stream) {
  if (dtype != PHS_F32 && dtype != PHS_F64) return PHS_ERR_DTYPE;
  if ((mid == nullptr) != (h1 == nullptr) || (h1 == nullptr) != (h2 == nullptr)) return PHS_ERR_INVALID;
  const int M = nb - 1 > na ? nb - 1 : na;
  if (B < 0 || T < 1 || nb < 1 || nb > 5 || na < 1 || na > 4 || padlen < 0 || padlen >= T ||
      padmode < PHS_PAD_CONSTANT || padmode > PHS_PAD_CIRCULAR)
    return PHS_ERR_INVALID;
  if ((grad_b == nullptr) != (grad_a == nullptr)) return PHS_ERR_INVALID;
  if (B == 0) return PHS_OK;
  if (!b || !a || !grad_y || !grad_x || (grad_b && !x)) return PHS_ERR_INVALID;
  const int64_t tile = dtype == PHS_F32 ? phs::SsShape<phs::Scalar<float>>::kTile : phs::SsShape<phs::Scalar<double>>::kTile;
  if (!phs::ss_grid_ok(B, T, tile)) return PHS_ERR_INVALID;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  phs::SsFilter f;
  f.b = b;
  f.a = a;
  f.nb = nb;
  f.na = na;
  f.form = 1;  // the forward's TDF-II model (ss_filtfilt_entry)
  f.shared = coef_shared != 0;
  return phs::ss_dispatch(dtype, M, [&](auto alg) {
    return phs::ss_filtfilt_bwd<decltype(alg)>(B, T, f, padmode, padlen, x, grad_y, grad_x, grad_b, grad_a, scratch,
                                               scratch_bytes, workspace, workspace_bytes, st, mid, h1, h2);
  });
}

}  // extern "C"
