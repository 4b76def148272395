// C ABI of the fused multi-input, multi-output LTI state space (declared in
// include/philscan.h): argument checks, workspace carving and the launch of
// mimo_ss_kernel on the caller's stream.  No allocation and no
// synchronisation.  Workspace layout: [0, 2048) claim header, then the status
// words of every (row, tile).
#include "phs_launch.hpp"
#include "phs_mimo.hpp"

namespace phs {
namespace {

template <class Alg>
size_t mimo_ws_bytes(int64_t B, int64_t T) {
  const int64_t tiles = (T + MimoShape<Alg>::kTile - 1) / MimoShape<Alg>::kTile;
  return align_up(align_up(kHeaderBytes) + size_t(B) * size_t(tiles) * StatusShape<Alg>::kStride * sizeof(uint64_t));
}

// ceil(2^32 / w): (e * magic) >> 32 == e / w for the element counts of a span
uint64_t io_magic(int w) { return ((uint64_t(1) << 32) + uint64_t(w) - 1) / uint64_t(w); }

// zf of an empty row: zi, or zeros
template <typename E>
__global__ __launch_bounds__(256) void mimo_empty_zf_kernel(const E *zi, int64_t n, E *zf) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) zf[i] = zi ? zi[i] : E(0);
}

template <class Alg>
int mimo_ss(int F, int P, int64_t B, int64_t T, const void *A, const void *Bm, const void *Cm, const void *Dm,
            int shared, const void *zi, const void *x, void *y, void *zf, void *workspace, size_t ws_bytes, bool rev,
            hipStream_t stream) {
  using E = typename Alg::elem;
  using Sh = MimoShape<Alg>;
  constexpr int M = SsView<Alg>::M;
  if (B < 0 || T < 0 || F < 1 || F > kMimoMaxIO || P < 1 || P > kMimoMaxIO) return PHS_ERR_INVALID;
  if (shared & ~(PHS_MIMO_A_SHARED | PHS_MIMO_B_SHARED | PHS_MIMO_C_SHARED | PHS_MIMO_D_SHARED))
    return PHS_ERR_INVALID;
  if (B == 0) return PHS_OK;
  if (T == 0) {
    if (zf) {
      const int64_t n = B * M;
      hipLaunchKernelGGL(mimo_empty_zf_kernel<E>, dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream,
                         static_cast<const E *>(zi), n, static_cast<E *>(zf));
      return hipGetLastError() == hipSuccess ? PHS_OK : PHS_ERR_LAUNCH;
    }
    return PHS_OK;
  }
  if (!A || !Bm || !Cm || !x || !y) return PHS_ERR_INVALID;
  const int64_t tiles_per_row = (T + Sh::kTile - 1) / Sh::kTile;
  if (double(B) * double(tiles_per_row) >= 2147483648.0) return PHS_ERR_INVALID;
  if (!workspace || ws_bytes < mimo_ws_bytes<Alg>(B, T)) return PHS_ERR_WORKSPACE;
  char *ws = static_cast<char *>(workspace);
  MimoArgs<Alg> a{};
  a.A = static_cast<const E *>(A);
  a.A_stride = (shared & PHS_MIMO_A_SHARED) ? 0 : M * M;
  a.Bm = static_cast<const E *>(Bm);
  a.b_stride = (shared & PHS_MIMO_B_SHARED) ? 0 : int64_t(M) * F;
  a.Cm = static_cast<const E *>(Cm);
  a.c_stride = (shared & PHS_MIMO_C_SHARED) ? 0 : int64_t(P) * M;
  a.Dm = static_cast<const E *>(Dm);
  a.d_stride = (shared & PHS_MIMO_D_SHARED) ? 0 : int64_t(P) * F;
  a.F = F;
  a.P = P;
  a.f_magic = io_magic(F);
  a.p_magic = io_magic(P);
  a.zi = static_cast<const E *>(zi);
  a.x = static_cast<const E *>(x);
  a.y = static_cast<E *>(y);
  a.zf = static_cast<E *>(zf);
  a.B = B;
  a.T_len = T;
  a.tiles_per_row = tiles_per_row;
  row_split(B, a.b_magic, a.b_shift);
  a.claims = reinterpret_cast<unsigned long long *>(ws);
  a.status = reinterpret_cast<uint64_t *>(ws + align_up(kHeaderBytes));
  a.tiles = unsigned(B * tiles_per_row);
  a.per_stripe = (a.tiles + kStripes - 1) / kStripes;
  const unsigned sl = g_spin_limit.load(std::memory_order_relaxed);
  a.spin_limit = sl ? sl : kDefaultSpinLimit;
  a.agg_only = g_agg_only.load(std::memory_order_relaxed) ? 1u : 0u;
  const dim3 grid(a.per_stripe * kStripes), block(Sh::kThreads);
  if (rev)
    launch_kernel((mimo_ss_kernel<Alg, true>), grid, block, 0, stream, a);
  else
    launch_kernel((mimo_ss_kernel<Alg, false>), grid, block, 0, stream, a);
  return hipGetLastError() == hipSuccess ? PHS_OK : PHS_ERR_LAUNCH;
}

template <class Fn>
int mimo_dispatch(int dtype, int M, Fn &&f) {
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

int mimo_call(int dtype, int M, int F, int P, int64_t B, int64_t T, const void *A, const void *Bm, const void *Cm,
              const void *Dm, int shared, const void *zi, const void *x, void *y, void *zf, void *workspace,
              size_t workspace_bytes, bool rev, void *stream) {
  const hipStream_t st = static_cast<hipStream_t>(stream);
  return mimo_dispatch(dtype, M, [&](auto alg) {
    return mimo_ss<decltype(alg)>(F, P, B, T, A, Bm, Cm, Dm, shared, zi, x, y, zf, workspace, workspace_bytes, rev,
                                  st);
  });
}

}  // namespace
}  // namespace phs

extern "C" {

size_t phs_mimo_ss_workspace_size(int dtype, int M, int64_t B, int64_t T) {
  if (B < 0 || T < 0) return 0;
  size_t out = 0;
  const int rc = phs::mimo_dispatch(dtype, M, [&](auto alg) {
    out = phs::mimo_ws_bytes<decltype(alg)>(B, T);
    return PHS_OK;
  });
  return rc == PHS_OK ? out : 0;
}

int phs_mimo_ss_fwd(int dtype, int M, int F, int P, int64_t B, int64_t T, const void *A, const void *Bm,
                    const void *Cm, const void *Dm, int shared, const void *zi, const void *x, void *y, void *zf,
                    void *workspace, size_t workspace_bytes, void *stream) {
  return phs::mimo_call(dtype, M, F, P, B, T, A, Bm, Cm, Dm, shared, zi, x, y, zf, workspace, workspace_bytes, false,
                        stream);
}

int phs_mimo_ss_rev(int dtype, int M, int F, int P, int64_t B, int64_t T, const void *A, const void *Bm,
                    const void *Cm, const void *Dm, int shared, const void *zi, const void *x, void *y, void *zf,
                    void *workspace, size_t workspace_bytes, void *stream) {
  return phs::mimo_call(dtype, M, F, P, B, T, A, Bm, Cm, Dm, shared, zi, x, y, zf, workspace, workspace_bytes, true,
                        stream);
}

}  // extern "C"
