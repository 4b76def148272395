// C ABI of the fused single-input, single-output LPV state space (declared in
// include/philscan.h): argument checks, workspace carving and the launch of
// lpv_ss_kernel on the caller's stream.  No allocation and no
// synchronisation.  Workspace layout: [0, 2048) claim header, then the status
// words of every (row, tile).
#include "phs_launch.hpp"
#include "phs_lpvss.hpp"

namespace phs {
namespace {

template <class Alg>
size_t lpv_ss_ws_bytes(int64_t B, int64_t T) {
  const int64_t tiles = (T + LpvSsShape<Alg>::kTile - 1) / LpvSsShape<Alg>::kTile;
  return align_up(align_up(kHeaderBytes) + size_t(B) * size_t(tiles) * StatusShape<Alg>::kStride * sizeof(uint64_t));
}

template <class Alg>
int lpv_ss_fwd(int64_t B, int64_t T, const void *A, bool A_sh, bool A_tr, LpvOperand<typename Alg::elem> bv,
               LpvOperand<typename Alg::elem> cv, int out_idx, LpvOperand<typename Alg::elem> d, const void *zi,
               const void *x, void *y, void *zf, void *workspace, size_t ws_bytes, bool rev, hipStream_t stream) {
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
  char *ws = static_cast<char *>(workspace);
  LpvSsArgs<Alg> a{};
  a.A = static_cast<const E *>(A);
  a.A_row_stride = A_sh ? 0 : T * M * M;
  a.A_trans = A_tr ? 1 : 0;
  a.bv = bv;
  a.cv = cv;
  a.d = d;
  a.out_idx = out_idx;
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
  a.vec_ok = (size_t(T) * sizeof(E)) % 16 == 0 && aligned16(x) && aligned16(y) && aligned16(A);
  if (rev)
    launch_kernel((lpv_ss_kernel<Alg, true>), dim3(a.per_stripe * kStripes), dim3(Sh::kThreads), 0, stream, a);
  else
    launch_kernel((lpv_ss_kernel<Alg, false>), dim3(a.per_stripe * kStripes), dim3(Sh::kThreads), 0, stream, a);
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
                void *y, void *zf, void *workspace, size_t workspace_bytes, bool rev, void *stream) {
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (A_flags & ~(PHS_LPV_A_SHARED | PHS_LPV_A_TRANSPOSED)) return PHS_ERR_INVALID;
  return phs::lpv_dispatch(dtype, M, [&](auto alg) {
    using E = typename decltype(alg)::elem;
    const phs::LpvOperand<E> bo{static_cast<const E *>(b), b_row_stride, b_t_stride};
    const phs::LpvOperand<E> co{static_cast<const E *>(c), c_row_stride, c_t_stride};
    const phs::LpvOperand<E> dd{static_cast<const E *>(d), d_row_stride, d_t_stride};
    return phs::lpv_ss_fwd<decltype(alg)>(B, T, A, (A_flags & PHS_LPV_A_SHARED) != 0,
                                          (A_flags & PHS_LPV_A_TRANSPOSED) != 0, bo, co, out_idx, dd, zi, x, y, zf,
                                          workspace, workspace_bytes, rev, st);
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

}  // extern "C"
