// C ABI of the fused single-input, single-output LTI state space (declared in
// include/philscan.h): argument checks, workspace carving and the launch of
// ss_kernel on the caller's stream.  No allocation and no synchronisation.
// Workspace layout: [0, 2048) claim header, then the status words of every
// (row, tile).
#include "phs_launch.hpp"
#include "phs_ss.hpp"

namespace phs {
namespace {

template <class Alg>
size_t ss_ws_bytes(int64_t B, int64_t T) {
  const int64_t tiles = (T + SsShape<Alg>::kTile - 1) / SsShape<Alg>::kTile;
  return align_up(align_up(kHeaderBytes) + size_t(B) * size_t(tiles) * SsStatus<Alg>::kStride * sizeof(uint64_t));
}

// Filter mode of the model (SsArgs::filt_form and friends): none, or
// lfilter(b, a) in companion form.
struct SsFilter {
  const void *b = nullptr, *a = nullptr;
  int nb = 0, na = 0, form = 0;
  bool shared = false;
};

template <class Alg>
int ss_fwd(int64_t B, int64_t T, const void *A, bool A_sh, const void *bv, bool b_sh, const void *cv, bool c_sh,
           int out_idx, const void *d, bool d_sh, const SsFilter &f, const void *zi, const void *x, void *y, void *zf,
           void *workspace, size_t ws_bytes, hipStream_t stream) {
  using E = typename Alg::elem;
  using Sh = SsShape<Alg>;
  constexpr int M = SsView<Alg>::M;
  if (B < 0 || T < 0) return PHS_ERR_INVALID;
  if (f.form == 0 && !cv && (out_idx < 0 || out_idx >= M)) return PHS_ERR_INVALID;
  if (f.form != 0 && (f.nb < 1 || f.nb > M + 1 || f.na < 1 || f.na > M || (f.nb - 1 != M && f.na != M)))
    return PHS_ERR_INVALID;
  if (B == 0 || T == 0) return PHS_OK;
  if ((f.form == 0 ? !A : (!f.b || !f.a)) || !x || !y) return PHS_ERR_INVALID;
  const int64_t tiles_per_row = (T + Sh::kTile - 1) / Sh::kTile;
  if (double(B) * double(tiles_per_row) >= 2147483648.0) return PHS_ERR_INVALID;
  if (!workspace || ws_bytes < ss_ws_bytes<Alg>(B, T)) return PHS_ERR_WORKSPACE;
  char *ws = static_cast<char *>(workspace);
  SsArgs<Alg> a{};
  a.A = static_cast<const E *>(A);
  a.A_stride = A_sh ? 0 : M * M;
  a.bv = static_cast<const E *>(bv);
  a.b_stride = b_sh ? 0 : M;
  a.cv = static_cast<const E *>(cv);
  a.c_stride = c_sh ? 0 : M;
  a.d = static_cast<const E *>(d);
  a.d_stride = d_sh ? 0 : 1;
  a.out_idx = out_idx;
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
  a.vec_ok = (size_t(T) * sizeof(E)) % 16 == 0 && aligned16(x) && aligned16(y);
  hipLaunchKernelGGL(ss_kernel<Alg>, dim3(a.per_stripe * kStripes), dim3(Sh::kThreads), 0, stream, a);
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

int phs_lti_ss_fwd(int dtype, int M, int64_t B, int64_t T, const void *A, int A_shared, const void *b, int b_shared,
                   const void *c, int c_shared, int out_idx, const void *d, int d_shared, const void *zi,
                   const void *x, void *y, void *zf, void *workspace, size_t workspace_bytes, void *stream) {
  const hipStream_t st = static_cast<hipStream_t>(stream);
  return phs::ss_dispatch(dtype, M, [&](auto alg) {
    return phs::ss_fwd<decltype(alg)>(B, T, A, A_shared != 0, b, b_shared != 0, c, c_shared != 0, out_idx, d,
                                      d_shared != 0, phs::SsFilter{}, zi, x, y, zf, workspace, workspace_bytes, st);
  });
}

int phs_lfilter_fwd(int dtype, int64_t B, int64_t T, const void *b, int nb, const void *a, int na, int coef_shared,
                    int form, const void *zi, const void *x, void *y, void *zf, void *workspace,
                    size_t workspace_bytes, void *stream) {
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
                                      x, y, zf, workspace, workspace_bytes, st);
  });
}

}  // extern "C"
