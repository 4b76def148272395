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
  return align_up(align_up(kHeaderBytes) + size_t(B) * size_t(tiles) * SsStatus<Alg>::kStride * sizeof(uint64_t));
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

// ---- sums over time of outer products (the coefficient gradients of the
// model: dL/dA = sum lambda h^T, dL/dB = sum lambda x^T, dL/dC = sum g h^T,
// dL/dD = sum g x^T).  A block sums `chunk` steps of one row: each thread
// its strided steps in compute precision, then the block through LDS, one
// partial per (row, block); the second kernel sums the partials in row and
// block order (and over the rows for a shared operand).
constexpr int kOuterThreads = 256;
constexpr int kOuterSteps = 64;  // steps per thread and block
constexpr int kOuterMax = kMimoMaxIO * kMimoMaxIO;

template <typename E>
__global__ __launch_bounds__(kOuterThreads) void mimo_outer_partial_kernel(const E *L, int nl, const E *R, int nr,
                                                                         int64_t T, typename Wide<E>::type *part) {
  using C = typename Wide<E>::type;
  __shared__ C s_red[kOuterThreads / 64][kOuterMax];
  const int64_t b = blockIdx.y, blk = blockIdx.x;
  const int64_t chunk = int64_t(kOuterThreads) * kOuterSteps;
  const int64_t t0 = blk * chunk, t1 = t0 + chunk < T ? t0 + chunk : T;
  const E *lrow = L + b * T * nl;
  const E *rrow = R + b * T * nr;
  C acc[kMimoMaxIO][kMimoMaxIO];
#pragma unroll
  for (int i = 0; i < kMimoMaxIO; ++i)
#pragma unroll
    for (int j = 0; j < kMimoMaxIO; ++j) acc[i][j] = C(0);
  for (int64_t t = t0 + threadIdx.x; t < t1; t += kOuterThreads) {
    E l[kMimoMaxIO], r[kMimoMaxIO];
#pragma unroll
    for (int i = 0; i < kMimoMaxIO; ++i) {
      l[i] = i < nl ? lrow[t * nl + i] : E(0);
      r[i] = i < nr ? rrow[t * nr + i] : E(0);
    }
#pragma unroll
    for (int i = 0; i < kMimoMaxIO; ++i)
#pragma unroll
      for (int j = 0; j < kMimoMaxIO; ++j) acc[i][j] = fma(C(l[i]), C(r[j]), acc[i][j]);
  }
  // the wave's sums by DPP scans, then the block's through LDS
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  auto add = [](const C &p, const C &o) { return p + o; };
#pragma unroll
  for (int i = 0; i < kMimoMaxIO; ++i)
#pragma unroll
    for (int j = 0; j < kMimoMaxIO; ++j) {
      const C v = read_lane(wave_scan_incl(acc[i][j], lane, add), 63);
      if (lane == 0) s_red[wv][i * kMimoMaxIO + j] = v;
    }
  __syncthreads();
  if (threadIdx.x < kOuterMax) {
    C v = C(0);
#pragma unroll
    for (int k = 0; k < kOuterThreads / 64; ++k) v += s_red[k][threadIdx.x];
    part[(b * gridDim.x + blk) * kOuterMax + threadIdx.x] = v;
  }
}

// out[row or 0][i][j] (i < nl, j < nr) from the partials of `blocks` blocks
// per row; shared: one sum over every row.  A block per output row, its
// threads strided over the partials, then the block's sums through LDS.
template <typename E>
__global__ __launch_bounds__(kOuterThreads) void mimo_outer_finish_kernel(const typename Wide<E>::type *part,
                                                                        int64_t rows, int64_t blocks, int nl, int nr,
                                                                        int shared, E *out) {
  using C = typename Wide<E>::type;
  __shared__ C s_red[kOuterThreads / 64][kOuterMax];
  const int64_t o = blockIdx.x;  // output row
  const int64_t p0 = shared ? 0 : o * blocks, n = shared ? rows * blocks : blocks;
  C acc[kOuterMax];
#pragma unroll
  for (int k = 0; k < kOuterMax; ++k) acc[k] = C(0);
  for (int64_t p = threadIdx.x; p < n; p += kOuterThreads) {
#pragma unroll
    for (int k = 0; k < kOuterMax; ++k) acc[k] += part[(p0 + p) * kOuterMax + k];
  }
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  auto add = [](const C &a, const C &b) { return a + b; };
#pragma unroll
  for (int k = 0; k < kOuterMax; ++k) {
    const C v = read_lane(wave_scan_incl(acc[k], lane, add), 63);
    if (lane == 0) s_red[wv][k] = v;
  }
  __syncthreads();
  const int i = threadIdx.x / kMimoMaxIO, j = threadIdx.x % kMimoMaxIO;
  if (threadIdx.x < kOuterMax && i < nl && j < nr) {
    C v = C(0);
#pragma unroll
    for (int k = 0; k < kOuterThreads / 64; ++k) v += s_red[k][threadIdx.x];
    out[(o * nl + i) * nr + j] = down<E>(v);
  }
}

template <typename E>
int outer_sums(int64_t B, int64_t T, const void *L, int nl, const void *R, int nr, int shared, void *out,
               void *scratch, size_t scratch_bytes, hipStream_t stream) {
  using C = typename Wide<E>::type;
  if (B < 0 || T < 0 || nl < 1 || nl > kMimoMaxIO || nr < 1 || nr > kMimoMaxIO || (shared & ~1)) return PHS_ERR_INVALID;
  if (!out) return PHS_ERR_INVALID;
  const int64_t orows = shared ? 1 : B;
  if (orows == 0) return PHS_OK;
  const int64_t chunk = int64_t(kOuterThreads) * kOuterSteps;
  const int64_t blocks = (T + chunk - 1) / chunk;
  if (B * blocks > 0) {
    if (!L || !R) return PHS_ERR_INVALID;
    if (B > 65535) return PHS_ERR_INVALID;
    if (!scratch || scratch_bytes < size_t(B) * size_t(blocks) * kOuterMax * sizeof(C)) return PHS_ERR_WORKSPACE;
    hipLaunchKernelGGL(mimo_outer_partial_kernel<E>, dim3(unsigned(blocks), unsigned(B)), dim3(kOuterThreads), 0,
                       stream, static_cast<const E *>(L), nl, static_cast<const E *>(R), nr, T,
                       static_cast<C *>(scratch));
  }
  hipLaunchKernelGGL(mimo_outer_finish_kernel<E>, dim3(unsigned(orows)), dim3(kOuterThreads), 0, stream,
                     static_cast<const C *>(scratch), B, blocks, nl, nr, shared, static_cast<E *>(out));
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

size_t phs_outer_sums_scratch_size(int dtype, int64_t B, int64_t T) {
  if (B < 0 || T < 0 || (dtype != PHS_F32 && dtype != PHS_F64)) return 0;
  const int64_t chunk = int64_t(phs::kOuterThreads) * phs::kOuterSteps;
  return size_t(B) * size_t((T + chunk - 1) / chunk) * phs::kOuterMax * sizeof(double);
}

int phs_outer_sums(int dtype, int64_t B, int64_t T, const void *L, int nl, const void *R, int nr, int shared,
                   void *out, void *scratch, size_t scratch_bytes, void *stream) {
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == PHS_F32) return phs::outer_sums<float>(B, T, L, nl, R, nr, shared, out, scratch, scratch_bytes, st);
  if (dtype == PHS_F64) return phs::outer_sums<double>(B, T, L, nl, R, nr, shared, out, scratch, scratch_bytes, st);
  return PHS_ERR_DTYPE;
}

}  // extern "C"
