// C ABI of the fused single-input, single-output LPV state space (declared in
// include/philscan.h): argument checks, workspace carving and the launch of
// lpv_ss_kernel on the caller's stream.  No allocation and no
// synchronisation.  Workspace layout: [0, 2048) claim header, then the status
// words of every (row, tile).  The coefficient-gradient backward takes a
// scratch buffer of its own: the forward's states, the per-wave sums, the
// row sums and the per-row, per-step gradients of operands the rows share.
#include "phs_launch.hpp"
#include "phs_lpvss.hpp"

namespace phs {
namespace {

template <class Alg>
size_t lpv_ss_ws_bytes(int64_t B, int64_t T) {
  const int64_t tiles = (T + LpvSsShape<Alg>::kTile - 1) / LpvSsShape<Alg>::kTile;
  return align_up(align_up(kHeaderBytes) + size_t(B) * size_t(tiles) * StatusShape<Alg>::kStride * sizeof(uint64_t));
}

// The launch arguments of one pass over [B, T] (the workspace carved as
// above; the caller has checked its size).
template <class Alg>
LpvSsArgs<Alg> lpv_args(int64_t B, int64_t T, const void *A, bool A_sh, bool A_tr, LpvOperand<typename Alg::elem> bv,
                        LpvOperand<typename Alg::elem> cv, int out_idx, int in_idx, LpvOperand<typename Alg::elem> d,
                        const void *zi, const void *x, void *y, void *zf, void *workspace) {
  using E = typename Alg::elem;
  using Sh = LpvSsShape<Alg>;
  constexpr int M = SsView<Alg>::M;
  char *ws = static_cast<char *>(workspace);
  const int64_t tiles_per_row = (T + Sh::kTile - 1) / Sh::kTile;
  LpvSsArgs<Alg> a{};
  a.A = static_cast<const E *>(A);
  a.A_row_stride = A_sh ? 0 : T * M * M;
  a.A_trans = A_tr ? 1 : 0;
  a.bv = bv;
  a.cv = cv;
  a.d = d;
  a.out_idx = out_idx;
  a.in_idx = in_idx;
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
  row_split(B, a.b_magic, a.b_shift);
  a.per_stripe = (a.tiles + kStripes - 1) / kStripes;
  const unsigned sl = g_spin_limit.load(std::memory_order_relaxed);
  a.spin_limit = sl ? sl : kDefaultSpinLimit;
  a.agg_only = g_agg_only.load(std::memory_order_relaxed) ? 1u : 0u;
  a.vec_ok = (size_t(T) * sizeof(E)) % 16 == 0 && aligned16(x) && aligned16(y) && aligned16(A);
  return a;
}

template <class Alg, bool REV, int MODE = kSsPlain>
int lpv_launch(const LpvSsArgs<Alg> &a, hipStream_t stream) {
  launch_kernel((lpv_ss_kernel<Alg, REV, MODE>), dim3(a.per_stripe * kStripes), dim3(LpvSsShape<Alg>::kThreads), 0,
                stream, a);
  return hipGetLastError() == hipSuccess ? PHS_OK : PHS_ERR_LAUNCH;
}

// hs (nullable): the state before every step [B, T, M] as well (the states
// the coefficient backward reads), written in the same pass as y.
template <class Alg>
int lpv_ss_fwd(int64_t B, int64_t T, const void *A, bool A_sh, bool A_tr, LpvOperand<typename Alg::elem> bv,
               LpvOperand<typename Alg::elem> cv, int out_idx, LpvOperand<typename Alg::elem> d, const void *zi,
               const void *x, void *y, void *zf, void *workspace, size_t ws_bytes, bool rev, hipStream_t stream,
               void *hs = nullptr) {
  using E = typename Alg::elem;
  using Sh = LpvSsShape<Alg>;
  constexpr int M = SsView<Alg>::M;
  if (B < 0 || T < 0) return PHS_ERR_INVALID;
  if (!cv.p && (out_idx < 0 || out_idx >= M)) return PHS_ERR_INVALID;
  for (const auto *o : {&bv, &cv, &d})
    if (o->row_stride < 0 || o->t_stride < 0) return PHS_ERR_INVALID;
  if (B == 0 || T == 0) return PHS_OK;
  if (!A || !x || !y) return PHS_ERR_INVALID;
  const int64_t tiles_per_row = (T + Sh::kTile - 1) / Sh::kTile;
  if (double(B) * double(tiles_per_row) >= 2147483648.0) return PHS_ERR_INVALID;
  if (!workspace || ws_bytes < lpv_ss_ws_bytes<Alg>(B, T)) return PHS_ERR_WORKSPACE;
  LpvSsArgs<Alg> a = lpv_args<Alg>(B, T, A, A_sh, A_tr, bv, cv, out_idx, 0, d, zi, x, y, zf, workspace);
  if (hs) {
    a.hs = static_cast<E *>(hs);
    a.vec_hs = aligned16(hs) && (size_t(T) * sizeof(typename Alg::s_state)) % 16 == 0 && aligned16(x) &&
               (size_t(T) * sizeof(E)) % 16 == 0;
    return rev ? lpv_launch<Alg, true, kSsStatesY>(a, stream) : lpv_launch<Alg, false, kSsStatesY>(a, stream);
  }
  return rev ? lpv_launch<Alg, true>(a, stream) : lpv_launch<Alg, false>(a, stream);
}

// Bits of the operands whose gradients vary along time and are shared by the
// rows (each takes a per-row scratch of its per-step gradients).
template <typename E>
int lpv_step_shared(bool A_sh, const LpvOperand<E> &bv, const LpvOperand<E> &cv, const LpvOperand<E> &d) {
  auto tv_shared = [](const LpvOperand<E> &o) { return o.p && o.row_stride == 0 && o.t_stride != 0; };
  return (A_sh ? PHS_LPV_GRAD_A : 0) | (tv_shared(bv) ? PHS_LPV_GRAD_B : 0) | (tv_shared(cv) ? PHS_LPV_GRAD_C : 0) |
         (tv_shared(d) ? PHS_LPV_GRAD_D : 0);
}

// The backward's scratch: states, per-wave sums, row sums, then the per-row
// per-step gradients of the operands in `step_shared` (A, b, c, d order).
template <class Alg>
struct LpvBwdLayout {
  size_t partials = 0, rowsum = 0, states = 0, step[4] = {0, 0, 0, 0}, total = 0;
};
template <class Alg>
LpvBwdLayout<Alg> lpv_bwd_layout(int64_t B, int64_t T, int step_shared) {
  using E = typename Alg::elem;
  using C = typename Wide<E>::type;
  constexpr int M = SsView<Alg>::M;
  const int64_t tiles = (T + LpvSsShape<Alg>::kTile - 1) / LpvSsShape<Alg>::kTile;
  LpvBwdLayout<Alg> L;
  size_t off = 0;
  L.states = off;
  off = align_up(off + size_t(B) * size_t(T) * sizeof(typename Alg::s_state));
  L.partials = off;
  off = align_up(off + size_t(B) * size_t(tiles) * LpvSsShape<Alg>::kWaves * SsGrad<Alg>::kN * sizeof(C));
  L.rowsum = off;
  off = align_up(off + size_t(B) * SsGrad<Alg>::kN * sizeof(C));
  const int width[4] = {M * M, M, M, 1};
  for (int i = 0; i < 4; ++i) {
    if (step_shared & (1 << i)) {
      L.step[i] = off;
      off = align_up(off + size_t(B) * size_t(T) * width[i] * sizeof(E));
    }
  }
  L.total = off;
  return L;
}

// Gradients of the model w.r.t. x, zi and A, b, c, d: the forward again
// writing its states (unless the forward gave them, hs_in), the adjoint model (A[t]^T, input vector c[t], output
// vector b[t], d[t]) in the opposite time direction from grad_zf with the
// coefficient gradients, the row sums of those constant in time and the
// batch sums of those the rows share.  The outputs are contiguous, shaped
// (1 | B, 1 | T, width) as their operands' sharing; each nullable.
template <class Alg>
int lpv_ss_bwd(int64_t B, int64_t T, const void *A, bool A_sh, bool A_tr, LpvOperand<typename Alg::elem> bv,
               LpvOperand<typename Alg::elem> cv, int out_idx, LpvOperand<typename Alg::elem> d, const void *zi,
               const void *x, const void *gy, const void *gzf, void *gx, void *gzi, void *gA, void *gb, void *gc,
               void *gd, void *scratch, size_t scratch_bytes, void *workspace, size_t ws_bytes, bool rev,
               hipStream_t stream, const void *hs_in = nullptr) {
  using E = typename Alg::elem;
  using C = typename Wide<E>::type;
  using SS = typename Alg::s_state;
  using Sh = LpvSsShape<Alg>;
  constexpr int M = SsView<Alg>::M;
  if (B < 0 || T < 0) return PHS_ERR_INVALID;
  if (!cv.p && (out_idx < 0 || out_idx >= M)) return PHS_ERR_INVALID;
  for (const auto *o : {&bv, &cv, &d})
    if (o->row_stride < 0 || o->t_stride < 0) return PHS_ERR_INVALID;
  if ((gb && !bv.p) || (gc && !cv.p) || (gd && !d.p)) return PHS_ERR_INVALID;
  if (B == 0) return PHS_OK;
  if (T > 0 && (!A || !x || !gy)) return PHS_ERR_INVALID;
  const int64_t tiles_per_row = (T + Sh::kTile - 1) / Sh::kTile;
  if (double(B) * double(tiles_per_row) >= 2147483648.0) return PHS_ERR_INVALID;
  const int shared = lpv_step_shared<E>(A_sh, bv, cv, d);
  const LpvBwdLayout<Alg> L = lpv_bwd_layout<Alg>(B, T, shared);
  if (!scratch || scratch_bytes < L.total) return PHS_ERR_WORKSPACE;
  if (T > 0 && (!workspace || ws_bytes < lpv_ss_ws_bytes<Alg>(B, T))) return PHS_ERR_WORKSPACE;
  char *sc = static_cast<char *>(scratch);
  E *states = hs_in ? const_cast<E *>(static_cast<const E *>(hs_in)) : reinterpret_cast<E *>(sc + L.states);
  C *gpart = reinterpret_cast<C *>(sc + L.partials);
  C *rowsum = reinterpret_cast<C *>(sc + L.rowsum);
  // where each per-step gradient goes: the output, or the per-row scratch
  E *outs[4] = {static_cast<E *>(gA), static_cast<E *>(gb), static_cast<E *>(gc), static_cast<E *>(gd)};
  const bool tv[4] = {true, bv.t_stride != 0, cv.t_stride != 0, d.t_stride != 0};
  E *step_dst[4];
  for (int i = 0; i < 4; ++i)
    step_dst[i] = (outs[i] && tv[i]) ? ((shared & (1 << i)) ? reinterpret_cast<E *>(sc + L.step[i]) : outs[i])
                                     : nullptr;
  const bool sum_b = gb && !tv[1], sum_c = gc && !tv[2], sum_d = gd && !tv[3];
  if (T > 0) {
    LpvSsArgs<Alg> p = lpv_args<Alg>(B, T, A, A_sh, A_tr, bv, cv, out_idx, 0, d, zi, x, nullptr, nullptr, workspace);
    p.hs = states;
    p.vec_hs = aligned16(states) && (size_t(T) * sizeof(SS)) % 16 == 0 && aligned16(x) &&
               (size_t(T) * sizeof(E)) % 16 == 0;
    int rc = PHS_OK;
    if (!hs_in) {
      rc = rev ? lpv_launch<Alg, true, kSsStates>(p, stream) : lpv_launch<Alg, false, kSsStates>(p, stream);
      if (rc != PHS_OK) return rc;
    }
    // the adjoint: A^T, input vector c (e_out_idx), output vector b (e_0)
    LpvSsArgs<Alg> q = lpv_args<Alg>(B, T, A, A_sh, !A_tr, cv, bv, 0, out_idx, d, gzf, gy, gx, gzi, workspace);
    q.hs_fwd = states;
    q.x_fwd = static_cast<const E *>(x);
    q.vec_hs = p.vec_hs;
    q.gA_step = step_dst[0];
    q.gb_step = step_dst[1];
    q.gc_step = step_dst[2];
    q.gd_step = step_dst[3];
    q.gA_trans = A_tr ? 1 : 0;
    q.sum_b = sum_b, q.sum_c = sum_c, q.sum_d = sum_d;
    q.gpart = (sum_b || sum_c || sum_d) ? gpart : nullptr;
    rc = rev ? lpv_launch<Alg, false, kSsGrad>(q, stream) : lpv_launch<Alg, true, kSsGrad>(q, stream);
    if (rc != PHS_OK) return rc;
  }
  // operands shared by the rows and varying along time: sums over the rows
  const int64_t width[4] = {M * M, M, M, 1};
  for (int i = 0; i < 4; ++i) {
    if (!(outs[i] && tv[i] && (shared & (1 << i))) || T == 0) continue;
    const int64_t n = T * width[i];
    const unsigned blocks = unsigned(std::min<int64_t>((n + 255) / 256, 4096));
    hipLaunchKernelGGL(lpv_grad_batch_kernel<E>, dim3(blocks), dim3(256), 0, stream,
                       static_cast<const E *>(step_dst[i]), B, n, outs[i]);
  }
  // operands constant in time (or T == 0): per-row sums, then the outputs
  // (a time-varying operand has no elements when T == 0)
  if (sum_b || sum_c || sum_d || T == 0) {
    SsGradOut<E> o{};
    o.gb = sum_b ? static_cast<E *>(gb) : nullptr;
    o.gc = sum_c ? static_cast<E *>(gc) : nullptr;
    o.gd = sum_d ? static_cast<E *>(gd) : nullptr;
    o.b_sh = bv.row_stride == 0, o.c_sh = cv.row_stride == 0, o.d_sh = d.row_stride == 0;
    o.gzi = T == 0 ? static_cast<E *>(gzi) : nullptr;
    o.gzf = static_cast<const E *>(gzf);
    hipLaunchKernelGGL(ss_grad_rows_kernel<Alg>, dim3(unsigned(B)), dim3(kSsReduceThreads), 0, stream,
                       static_cast<const C *>(gpart), T == 0 ? int64_t(0) : tiles_per_row * Sh::kWaves, rowsum);
    hipLaunchKernelGGL(ss_grad_finish_kernel<Alg>, dim3(1), dim3(kSsReduceThreads), 0, stream,
                       static_cast<const C *>(rowsum), B, T, o);
  }
  return hipGetLastError() == hipSuccess ? PHS_OK : PHS_ERR_LAUNCH;
}

template <class F>
int lpv_dispatch(int dtype, int M, F &&f) {
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
}  // namespace phs

extern "C" {

size_t phs_lpv_ss_bwd_scratch_size(int dtype, int M, int64_t B, int64_t T, int step_shared) {
  if (B < 0 || T < 0 || (step_shared & ~15)) return 0;
  size_t out = 0;
  const int rc = phs::lpv_dispatch(dtype, M, [&](auto alg) {
    out = phs::lpv_bwd_layout<decltype(alg)>(B, T, step_shared).total;
    return PHS_OK;
  });
  return rc == PHS_OK ? out : 0;
}

int phs_lpv_ss_bwd(int dtype, int M, int64_t B, int64_t T, const void *A, int A_flags, const void *b,
                   int64_t b_row_stride, int64_t b_t_stride, const void *c, int64_t c_row_stride, int64_t c_t_stride,
                   int out_idx, const void *d, int64_t d_row_stride, int64_t d_t_stride, const void *zi,
                   const void *x, const void *gy, const void *gzf, void *gx, void *gzi, void *gA, void *gb, void *gc,
                   void *gd, int reverse, void *scratch, size_t scratch_bytes, void *workspace,
                   size_t workspace_bytes, void *stream) {
  return phs_lpv_ss_bwd_hs(dtype, M, B, T, A, A_flags, b, b_row_stride, b_t_stride, c, c_row_stride, c_t_stride,
                           out_idx, d, d_row_stride, d_t_stride, zi, x, nullptr, gy, gzf, gx, gzi, gA, gb, gc, gd,
                           reverse, scratch, scratch_bytes, workspace, workspace_bytes, stream);
}

int phs_lpv_ss_bwd_hs(int dtype, int M, int64_t B, int64_t T, const void *A, int A_flags, const void *b,
                      int64_t b_row_stride, int64_t b_t_stride, const void *c, int64_t c_row_stride,
                      int64_t c_t_stride, int out_idx, const void *d, int64_t d_row_stride, int64_t d_t_stride,
                      const void *zi, const void *x, const void *hs, const void *gy, const void *gzf, void *gx,
                      void *gzi, void *gA, void *gb, void *gc, void *gd, int reverse, void *scratch,
                      size_t scratch_bytes, void *workspace, size_t workspace_bytes, void *stream) {
  if (A_flags & ~(PHS_LPV_A_SHARED | PHS_LPV_A_TRANSPOSED)) return PHS_ERR_INVALID;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  return phs::lpv_dispatch(dtype, M, [&](auto alg) {
    using E = typename decltype(alg)::elem;
    const phs::LpvOperand<E> bo{static_cast<const E *>(b), b_row_stride, b_t_stride};
    const phs::LpvOperand<E> co{static_cast<const E *>(c), c_row_stride, c_t_stride};
    const phs::LpvOperand<E> dd{static_cast<const E *>(d), d_row_stride, d_t_stride};
    return phs::lpv_ss_bwd<decltype(alg)>(B, T, A, (A_flags & PHS_LPV_A_SHARED) != 0,
                                          (A_flags & PHS_LPV_A_TRANSPOSED) != 0, bo, co, out_idx, dd, zi, x, gy, gzf,
                                          gx, gzi, gA, gb, gc, gd, scratch, scratch_bytes, workspace, workspace_bytes,
                                          reverse != 0, st, hs);
  });
}

size_t phs_lpv_ss_workspace_size(int dtype, int M, int64_t B, int64_t T) {
  if (B < 0 || T < 0) return 0;
  size_t out = 0;
  const int rc = phs::lpv_dispatch(dtype, M, [&](auto alg) {
    out = phs::lpv_ss_ws_bytes<decltype(alg)>(B, T);
    return PHS_OK;
  });
  return rc == PHS_OK ? out : 0;
}

namespace {

int lpv_ss_call(int dtype, int M, int64_t B, int64_t T, const void *A, int A_flags, const void *b,
                int64_t b_row_stride, int64_t b_t_stride, const void *c, int64_t c_row_stride, int64_t c_t_stride,
                int out_idx, const void *d, int64_t d_row_stride, int64_t d_t_stride, const void *zi, const void *x,
                void *y, void *zf, void *workspace, size_t workspace_bytes, bool rev, void *stream,
                void *hs = nullptr) {
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (A_flags & ~(PHS_LPV_A_SHARED | PHS_LPV_A_TRANSPOSED)) return PHS_ERR_INVALID;
  return phs::lpv_dispatch(dtype, M, [&](auto alg) {
    using E = typename decltype(alg)::elem;
    const phs::LpvOperand<E> bo{static_cast<const E *>(b), b_row_stride, b_t_stride};
    const phs::LpvOperand<E> co{static_cast<const E *>(c), c_row_stride, c_t_stride};
    const phs::LpvOperand<E> dd{static_cast<const E *>(d), d_row_stride, d_t_stride};
    return phs::lpv_ss_fwd<decltype(alg)>(B, T, A, (A_flags & PHS_LPV_A_SHARED) != 0,
                                          (A_flags & PHS_LPV_A_TRANSPOSED) != 0, bo, co, out_idx, dd, zi, x, y, zf,
                                          workspace, workspace_bytes, rev, st, hs);
  });
}

}  // namespace

int phs_lpv_ss_fwd(int dtype, int M, int64_t B, int64_t T, const void *A, int A_flags, const void *b,
                   int64_t b_row_stride, int64_t b_t_stride, const void *c, int64_t c_row_stride, int64_t c_t_stride,
                   int out_idx, const void *d, int64_t d_row_stride, int64_t d_t_stride, const void *zi,
                   const void *x, void *y, void *zf, void *workspace, size_t workspace_bytes, void *stream) {
  return lpv_ss_call(dtype, M, B, T, A, A_flags, b, b_row_stride, b_t_stride, c, c_row_stride, c_t_stride, out_idx,
                     d, d_row_stride, d_t_stride, zi, x, y, zf, workspace, workspace_bytes, false, stream);
}

int phs_lpv_ss_rev(int dtype, int M, int64_t B, int64_t T, const void *A, int A_flags, const void *b,
                   int64_t b_row_stride, int64_t b_t_stride, const void *c, int64_t c_row_stride, int64_t c_t_stride,
                   int out_idx, const void *d, int64_t d_row_stride, int64_t d_t_stride, const void *zi,
                   const void *x, void *y, void *zf, void *workspace, size_t workspace_bytes, void *stream) {
  return lpv_ss_call(dtype, M, B, T, A, A_flags, b, b_row_stride, b_t_stride, c, c_row_stride, c_t_stride, out_idx,
                     d, d_row_stride, d_t_stride, zi, x, y, zf, workspace, workspace_bytes, true, stream);
}

int phs_lpv_ss_fwd_hs(int dtype, int M, int64_t B, int64_t T, const void *A, int A_flags, const void *b,
                      int64_t b_row_stride, int64_t b_t_stride, const void *c, int64_t c_row_stride,
                      int64_t c_t_stride, int out_idx, const void *d, int64_t d_row_stride, int64_t d_t_stride,
                      const void *zi, const void *x, void *y, void *zf, void *hs, int reverse, void *workspace,
                      size_t workspace_bytes, void *stream) {
  if (!hs && B > 0 && T > 0) return PHS_ERR_INVALID;
  return lpv_ss_call(dtype, M, B, T, A, A_flags, b, b_row_stride, b_t_stride, c, c_row_stride, c_t_stride, out_idx,
                     d, d_row_stride, d_t_stride, zi, x, y, zf, workspace, workspace_bytes, reverse != 0, stream, hs);
}

}  // extern "C"
