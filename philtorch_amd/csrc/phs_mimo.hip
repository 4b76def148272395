// C ABI of the fused multi-input, multi-output state spaces, LTI and LPV
// (declared in include/philscan.h): argument checks, workspace carving and
// the launches of mimo_ss_kernel and lpv_mimo_kernel on the caller's stream.  No allocation and no
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

// ---- the coefficient gradients, summed over time in one pass over the
// forward's states h, the adjoint states lambda, x and g:
//   dL/dA = sum lambda h^T (M x M), dL/dB = sum lambda x^T (M x F),
//   dL/dC = sum g h^T (P x M),      dL/dD = sum g x^T (P x F),
// each wanted or not.  A block sums `chunk` steps of one row: each thread its
// strided steps in compute precision, then the block through LDS, one
// partial (the four products as 4 x 4 blocks) per (row, block); the second
// kernel sums each row's partials, the third the row totals of a product
// shared by the rows, each in a fixed order.  (Four separate sums of one product each read lambda, h,
// x and g twice: 372 against 93 us for one of them at the c4_mimo shape.)
constexpr int kSumThreads = 256;
constexpr int kSumSteps = 64;  // steps per thread and block
constexpr int kSumBlock = kMimoMaxIO * kMimoMaxIO;
constexpr int kSumN = 4 * kSumBlock;  // A, B, C, D

template <typename E>
struct GradSumIn {
  const E *lam, *hs, *x, *g;  // [B, T, M], [B, T, M], [B, T, F], [B, T, P]
  int M, F, P;
  unsigned want;  // bit i: product i (A, B, C, D)
  E *a_steps;     // non-null: lambda h^T per step [B, T, M, M] here, A not summed
  int a_trans;    // a_steps holds h lambda^T
  int a_vec;      // a_steps is 16-byte aligned
  // non-null gx: B^T lambda[t] + D^T g[t] per step [B, T, F] (the input's
  // gradient); Bm [B|1, M, F], Dm [B|1, P, F] or null, row strides 0 when shared
  E *gx;
  const E *Bm, *Dm;
  int64_t b_stride, d_stride;
};

// One step's operands in compute precision: lambda and h padded to WM with
// zeros, x and g to WI.
template <typename C, int WM, int WI>
struct SumStep {
  C l[WM], h[WM], u[WI], g[WI];
};

// The partial kernel at padded widths WM >= M (the state) and WI >= F, P
// (the input and output): the four products' accumulators take WM^2 +
// 2 WM WI + WI^2 registers (16 doubles at WM = WI = 2; padding every model
// to 4 took 64 and 180 VGPRs, two waves per SIMD: 717 us at the C3 shape),
// and each thread keeps U steps' loads in flight per iteration.  (Staging
// a block's steps through LDS with two barriers per 256 steps measured
// slower still: 1111 us.)
template <typename E, int WM, int WI, bool ALL>
__global__ __launch_bounds__(kSumThreads) void mimo_grad_partial_kernel(GradSumIn<E> in, int64_t T, unsigned nblk,
                                                                        typename Wide<E>::type *part) {
  using C = typename Wide<E>::type;
  constexpr int U = WM + WI <= 6 ? 4 : 2;
  __shared__ C s_red[kSumThreads / 64][kSumN];
  __shared__ C s_bd[2 * kSumBlock];  // gx: this row's B (M x F), then D (P x F), zero past them
  // one workgroup per (row, block of steps), row-major
  const int64_t b = blockIdx.x / nblk, blk = blockIdx.x - unsigned(b) * nblk;
  const int64_t chunk = int64_t(kSumThreads) * kSumSteps;
  const int64_t t0 = blk * chunk, t1 = t0 + chunk < T ? t0 + chunk : T;
  const int M = in.M, F = in.F, P = in.P;
  const bool wA = in.want & 1, wB = in.want & 2, wC = in.want & 4, wD = in.want & 8, wx = in.gx != nullptr;
  const bool need_l = wA || wB || wx, need_h = wA || wC, need_x = wB || wD, need_g = wC || wD || wx;
  const E *__restrict__ lrow = need_l ? in.lam + b * T * M : nullptr;
  const E *__restrict__ hrow = need_h ? in.hs + b * T * M : nullptr;
  const E *__restrict__ xrow = need_x ? in.x + b * T * F : nullptr;
  const E *__restrict__ grow = need_g ? in.g + b * T * P : nullptr;
  auto load = [&](int64_t t, SumStep<C, WM, WI> &s) {
    if constexpr (ALL) {
      // every operand there: unconditional loads (an index past the width
      // reads its last element, zeroed after), so a thread's U steps of
      // loads are all in flight before the first use
      E l[WM], h[WM], u[WI], g[WI];
#pragma unroll
      for (int i = 0; i < WM; ++i) {
        l[i] = lrow[t * M + (i < M ? i : M - 1)];
        h[i] = hrow[t * M + (i < M ? i : M - 1)];
      }
#pragma unroll
      for (int i = 0; i < WI; ++i) {
        u[i] = xrow[t * F + (i < F ? i : F - 1)];
        g[i] = grow[t * P + (i < P ? i : P - 1)];
      }
#pragma unroll
      for (int i = 0; i < WM; ++i) {
        s.l[i] = i < M ? C(l[i]) : C(0);
        s.h[i] = i < M ? C(h[i]) : C(0);
      }
#pragma unroll
      for (int i = 0; i < WI; ++i) {
        s.u[i] = i < F ? C(u[i]) : C(0);
        s.g[i] = i < P ? C(g[i]) : C(0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < WM; ++i) {
        s.l[i] = s.h[i] = C(0);
        if (need_l && i < M) s.l[i] = C(lrow[t * M + i]);
        if (need_h && i < M) s.h[i] = C(hrow[t * M + i]);
      }
#pragma unroll
      for (int i = 0; i < WI; ++i) {
        s.u[i] = s.g[i] = C(0);
        if (need_x && i < F) s.u[i] = C(xrow[t * F + i]);
        if (need_g && i < P) s.g[i] = C(grow[t * P + i]);
      }
    }
  };
  C aA[WM][WM], aB[WM][WI], aC[WI][WM], aD[WI][WI];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WM; ++j) aA[i][j] = C(0);
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WI; ++j) aB[i][j] = aC[j][i] = C(0);
#pragma unroll
  for (int i = 0; i < WI; ++i)
#pragma unroll
    for (int j = 0; j < WI; ++j) aD[i][j] = C(0);
  E *const arow = in.a_steps ? in.a_steps + b * T * M * M : nullptr;
  E *const gxrow = in.gx ? in.gx + b * T * F : nullptr;
  if (in.gx) {
    if (threadIdx.x < 2 * kSumBlock) {
      const int k = threadIdx.x % kSumBlock;
      C v = C(0);
      if (threadIdx.x < kSumBlock && k < M * F) v = C(in.Bm[b * in.b_stride + k]);
      if (threadIdx.x >= kSumBlock && in.Dm && k < P * F) v = C(in.Dm[b * in.d_stride + k]);
      s_bd[threadIdx.x] = v;
    }
    __syncthreads();
  }
  auto add_sums = [&](const SumStep<C, WM, WI> &s) {
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WM; ++j) aA[i][j] = fma(s.l[i], s.h[j], aA[i][j]);
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WI; ++j) {
        aB[i][j] = fma(s.l[i], s.u[j], aB[i][j]);
        aC[j][i] = fma(s.g[j], s.h[i], aC[j][i]);
      }
#pragma unroll
    for (int i = 0; i < WI; ++i)
#pragma unroll
      for (int j = 0; j < WI; ++j) aD[i][j] = fma(s.g[i], s.u[j], aD[i][j]);
  };
  auto add_step = [&](const SumStep<C, WM, WI> &s, int64_t t) {
    if (gxrow) {
      // the input's gradient, rounded once: lambda and g are zero past M
      // and P, and so are the entries of B and D past them
#pragma unroll
      for (int f = 0; f < WI; ++f) {
        if (f >= F) break;
        C v = C(0);
#pragma unroll
        for (int m = 0; m < WM; ++m) v = fma(s_bd[m * F + f], s.l[m], v);
#pragma unroll
        for (int q = 0; q < WI; ++q) v = fma(s_bd[kSumBlock + q * F + f], s.g[q], v);
        gxrow[t * F + f] = down<E>(v);
      }
    }
    if (arow) {
      // the per-step product, rounded once (exact in compute precision);
      // M = WM here.  A step's block in 16-byte stores where it is a whole
      // number of them and the buffer 16-byte aligned
      E v[WM * WM];  // compile-time indices on both branches: registers, not scratch
      if (in.a_trans) {
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
          for (int j = 0; j < WM; ++j) v[j * WM + i] = down<E>(s.l[i] * s.h[j]);
      } else {
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
          for (int j = 0; j < WM; ++j) v[i * WM + j] = down<E>(s.l[i] * s.h[j]);
      }
      E *dst = arow + t * WM * WM;
      constexpr int kPer16 = 16 / int(sizeof(E));
      if constexpr ((WM * WM) % kPer16 == 0) {
        using V16 = typename std::conditional<sizeof(E) == 4, float4, double2>::type;
        if (in.a_vec) {
#pragma unroll
          for (int k = 0; k < WM * WM / kPer16; ++k) {
            V16 w;
            __builtin_memcpy(&w, v + k * kPer16, 16);
            reinterpret_cast<V16 *>(dst)[k] = w;
          }
          return add_sums(s);
        }
      }
#pragma unroll
      for (int k = 0; k < WM * WM; ++k) dst[k] = v[k];
    }
    add_sums(s);
  };
  int64_t t = t0 + threadIdx.x;
  for (; t + (U - 1) * kSumThreads < t1; t += U * kSumThreads) {
    SumStep<C, WM, WI> s[U];
#pragma unroll
    for (int k = 0; k < U; ++k) load(t + k * kSumThreads, s[k]);
#pragma unroll
    for (int k = 0; k < U; ++k) add_step(s[k], t + k * kSumThreads);
  }
  for (; t < t1; t += kSumThreads) {
    SumStep<C, WM, WI> s;
    load(t, s);
    add_step(s, t);
  }
  // the wave's sums by DPP scans, then the block's through LDS (entries
  // past W: zeros)
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  auto add = [](const C &p, const C &o) { return p + o; };
  if (lane < kSumN) s_red[wv][lane] = C(0);
  auto put = [&](int p, int i, int j, const C &a) {
    const C v = read_lane(wave_scan_incl(a, lane, add), 63);
    if (lane == 0) s_red[wv][p * kSumBlock + i * kMimoMaxIO + j] = v;
  };
  if (wA && !arow)
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WM; ++j) put(0, i, j, aA[i][j]);
  if (wB)
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WI; ++j) put(1, i, j, aB[i][j]);
  if (wC)
#pragma unroll
    for (int i = 0; i < WI; ++i)
#pragma unroll
      for (int j = 0; j < WM; ++j) put(2, i, j, aC[i][j]);
  if (wD)
#pragma unroll
    for (int i = 0; i < WI; ++i)
#pragma unroll
      for (int j = 0; j < WI; ++j) put(3, i, j, aD[i][j]);
  __syncthreads();
  const unsigned summed = arow ? in.want & ~1u : in.want;
  if (threadIdx.x < kSumN && ((summed >> (threadIdx.x / kSumBlock)) & 1)) {
    C v = C(0);
#pragma unroll
    for (int k = 0; k < kSumThreads / 64; ++k) v += s_red[k][threadIdx.x];
    part[(b * nblk + blk) * kSumN + threadIdx.x] = v;
  }
}

template <typename E>
struct GradSumOut {
  E *out[4];      // A [B|1, M, M], B [B|1, M, F], C [B|1, P, M], D [B|1, P, F]; nullptr: not wanted
  int rows[4], cols[4];
  int shared;     // bit i: product i summed over the rows too
};

// Block r: row r's partials summed, thread (entry k, lane group q0) over
// every fourth partial (coalesced: a wave reads 64 consecutive entries),
// then the four groups through LDS.  A product not summed over the rows is
// written out; a shared one leaves the row's total in `rows` for the next
// kernel.  (One block summing a shared product over every row's partials
// took 66 us at the C3 shape.)
template <typename E>
__global__ __launch_bounds__(kSumThreads) void mimo_grad_rows_kernel(const typename Wide<E>::type *part,
                                                                     int64_t blocks, GradSumOut<E> o,
                                                                     typename Wide<E>::type *rows) {
  using C = typename Wide<E>::type;
  constexpr int G = kSumThreads / kSumN;
  __shared__ C s_red[G][kSumN];
  const int64_t r = blockIdx.x;
  const int k = threadIdx.x % kSumN, q0 = threadIdx.x / kSumN;
  const C *src = part + r * blocks * kSumN + k;
  C v[4] = {C(0), C(0), C(0), C(0)};
  int64_t q = q0;
  for (; q + 3 * G < blocks; q += 4 * G) {
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] += src[(q + u * G) * kSumN];
  }
  for (; q < blocks; q += G) v[0] += src[q * kSumN];
  s_red[q0][k] = (v[0] + v[1]) + (v[2] + v[3]);
  __syncthreads();
  if (threadIdx.x >= kSumN) return;
  C t = C(0);
#pragma unroll
  for (int w = 0; w < G; ++w) t += s_red[w][k];
  const int p = k / kSumBlock, i = (k % kSumBlock) / kMimoMaxIO, j = k % kMimoMaxIO;
  if (!o.out[p] || i >= o.rows[p] || j >= o.cols[p]) return;
  if ((o.shared >> p) & 1)
    rows[r * kSumN + k] = t;
  else
    o.out[p][(r * o.rows[p] + i) * o.cols[p] + j] = down<E>(t);
}

// One block: the shared products, the row totals summed by thread (entry
// k, row group q0) over every G-th row, then the groups through LDS.
constexpr int kSharedThreads = 1024;

template <typename E>
__global__ __launch_bounds__(kSharedThreads) void mimo_grad_shared_kernel(const typename Wide<E>::type *rows,
                                                                          int64_t B, GradSumOut<E> o) {
  using C = typename Wide<E>::type;
  constexpr int G = kSharedThreads / kSumN;
  __shared__ C s_red[G][kSumN];
  const int k = threadIdx.x % kSumN, q0 = threadIdx.x / kSumN;
  const int p = k / kSumBlock, i = (k % kSumBlock) / kMimoMaxIO, j = k % kMimoMaxIO;
  const bool mine = o.out[p] && ((o.shared >> p) & 1) && i < o.rows[p] && j < o.cols[p];
  C v[4] = {C(0), C(0), C(0), C(0)};
  if (mine) {
    int64_t q = q0;
    for (; q + 3 * G < B; q += 4 * G) {
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] += rows[(q + u * G) * kSumN + k];
    }
    for (; q < B; q += G) v[0] += rows[q * kSumN + k];
  }
  s_red[q0][k] = (v[0] + v[1]) + (v[2] + v[3]);
  __syncthreads();
  if (threadIdx.x >= kSumN || !mine) return;
  C t = C(0);
#pragma unroll
  for (int w = 0; w < G; ++w) t += s_red[w][k];
  o.out[p][i * o.cols[p] + j] = down<E>(t);
}

template <typename E>
int grad_sums(int M, int F, int P, int64_t B, int64_t T, const void *lam, const void *hs, const void *x,
              const void *g, const void *Bm, const void *Dm, int shared, void *gA, void *gB, void *gC, void *gD,
              void *gx, void *scratch, size_t scratch_bytes, hipStream_t stream) {
  using C = typename Wide<E>::type;
  if (B < 0 || T < 0 || M < 1 || M > kMimoMaxIO || F < 1 || F > kMimoMaxIO || P < 1 || P > kMimoMaxIO)
    return PHS_ERR_INVALID;
  if (shared & ~(PHS_MIMO_A_SHARED | PHS_MIMO_B_SHARED | PHS_MIMO_C_SHARED | PHS_MIMO_D_SHARED | PHS_MIMO_A_STEPS |
                 PHS_MIMO_A_STEPS_T))
    return PHS_ERR_INVALID;
  const bool steps = shared & PHS_MIMO_A_STEPS;
  if ((steps && (shared & PHS_MIMO_A_SHARED)) || (!steps && (shared & PHS_MIMO_A_STEPS_T))) return PHS_ERR_INVALID;
  GradSumIn<E> in{static_cast<const E *>(lam), static_cast<const E *>(hs), static_cast<const E *>(x),
                  static_cast<const E *>(g), M, F, P, 0u, nullptr, (shared & PHS_MIMO_A_STEPS_T) ? 1 : 0, 0};
  GradSumOut<E> o{};
  void *outs[4] = {steps ? nullptr : gA, gB, gC, gD};
  const int rows[4] = {M, M, P, P}, cols[4] = {M, F, M, F};
  for (int p = 0; p < 4; ++p) {
    o.out[p] = static_cast<E *>(outs[p]);
    o.rows[p] = rows[p];
    o.cols[p] = cols[p];
    if (outs[p]) in.want |= 1u << p;
  }
  if (steps && gA) {
    in.want |= 1u;  // reads lambda and h
    in.a_steps = static_cast<E *>(gA);
    in.a_vec = aligned16(gA);
  }
  if (gx) {
    if (!Bm) return PHS_ERR_INVALID;
    in.gx = static_cast<E *>(gx);
    in.Bm = static_cast<const E *>(Bm);
    in.Dm = static_cast<const E *>(Dm);
    in.b_stride = (shared & PHS_MIMO_B_SHARED) ? 0 : int64_t(M) * F;
    in.d_stride = (shared & PHS_MIMO_D_SHARED) ? 0 : int64_t(P) * F;
  }
  o.shared = shared & 15;
  if ((!in.want && !gx) || B == 0) return PHS_OK;
  const bool need_l = (in.want & 3) || gx, need_h = in.want & 5, need_x = in.want & 10, need_g = (in.want & 12) || gx;
  if (T > 0 && ((need_l && !lam) || (need_h && !hs) || (need_x && !x) || (need_g && !g))) return PHS_ERR_INVALID;
  const int64_t chunk = int64_t(kSumThreads) * kSumSteps;
  const int64_t blocks = (T + chunk - 1) / chunk;
  if (double(B) * double(blocks) >= 2147483648.0 || B >= 2147483648LL) return PHS_ERR_INVALID;
  if (!scratch || scratch_bytes < size_t(B) * size_t(blocks + 1) * kSumN * sizeof(C)) return PHS_ERR_WORKSPACE;
  if (blocks > 0) {
    // the state's width exact, the input's and output's rounded to 2 or 4;
    // all: the wanted products read every one of lambda, h, x and g
    const int WI = (F > P ? F : P) <= 2 ? 2 : 4;
    const bool all = need_l && need_h && need_x && need_g;
    auto pick = [&](auto wm) {
      constexpr int WMc = decltype(wm)::value;
      if (WI == 2) return all ? mimo_grad_partial_kernel<E, WMc, 2, true> : mimo_grad_partial_kernel<E, WMc, 2, false>;
      return all ? mimo_grad_partial_kernel<E, WMc, 4, true> : mimo_grad_partial_kernel<E, WMc, 4, false>;
    };
    auto kern = M == 1   ? pick(std::integral_constant<int, 1>{})
                : M == 2 ? pick(std::integral_constant<int, 2>{})
                : M == 3 ? pick(std::integral_constant<int, 3>{})
                         : pick(std::integral_constant<int, 4>{});
    hipLaunchKernelGGL(kern, dim3(unsigned(B * blocks)), dim3(kSumThreads), 0, stream, in, T, unsigned(blocks),
                       static_cast<C *>(scratch));
  }
  C *part = static_cast<C *>(scratch), *row_tot = part + B * blocks * kSumN;
  hipLaunchKernelGGL(mimo_grad_rows_kernel<E>, dim3(unsigned(B)), dim3(kSumThreads), 0, stream, part, blocks, o,
                     row_tot);
  bool any_shared = false;
  for (int p = 0; p < 4; ++p) any_shared |= o.out[p] && ((shared >> p) & 1);
  if (any_shared)
    hipLaunchKernelGGL(mimo_grad_shared_kernel<E>, dim3(1), dim3(kSharedThreads), 0, stream, row_tot, B, o);
  return hipGetLastError() == hipSuccess ? PHS_OK : PHS_ERR_LAUNCH;
}

// ---- the time-varying model (lpv_mimo_kernel)
template <class Alg>
size_t lpv_mimo_ws_bytes(int64_t B, int64_t T) {
  const int64_t tiles = (T + LpvMimoShape<Alg>::kTile - 1) / LpvMimoShape<Alg>::kTile;
  return align_up(align_up(kHeaderBytes) + size_t(B) * size_t(tiles) * StatusShape<Alg>::kStride * sizeof(uint64_t));
}

template <class Alg>
int lpv_mimo_ss(int F, int P, int64_t B, int64_t T, const void *A, int A_flags, const void *Bm, const void *Cm,
                const void *Dm, int shared, const void *zi, const void *x, void *y, void *zf, void *workspace,
                size_t ws_bytes, bool rev, hipStream_t stream, void *hs = nullptr) {
  using E = typename Alg::elem;
  using Sh = LpvMimoShape<Alg>;
  constexpr int M = SsView<Alg>::M;
  if (B < 0 || T < 0 || F < 1 || F > kMimoMaxIO || P < 1 || P > kMimoMaxIO) return PHS_ERR_INVALID;
  if (hs && P + M > kMimoMaxIO) return PHS_ERR_INVALID;  // the states share the outputs' LDS planes
  if ((shared & ~(PHS_MIMO_B_SHARED | PHS_MIMO_C_SHARED | PHS_MIMO_D_SHARED)) ||
      (A_flags & ~(PHS_LPV_A_SHARED | PHS_LPV_A_TRANSPOSED)))
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
  if (!workspace || ws_bytes < lpv_mimo_ws_bytes<Alg>(B, T)) return PHS_ERR_WORKSPACE;
  char *ws = static_cast<char *>(workspace);
  MimoArgs<Alg> a{};
  a.A = static_cast<const E *>(A);
  a.A_stride = (A_flags & PHS_LPV_A_SHARED) ? 0 : T * M * M;
  a.A_trans = (A_flags & PHS_LPV_A_TRANSPOSED) ? 1 : 0;
  a.A_vec = aligned16(A) && (size_t(T) * M * M * sizeof(E)) % 16 == 0;
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
  a.hs = static_cast<E *>(hs);
  a.m_magic = io_magic(M);
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
  if (hs) {
    if (rev)
      launch_kernel((lpv_mimo_kernel<Alg, true, true>), grid, block, 0, stream, a);
    else
      launch_kernel((lpv_mimo_kernel<Alg, false, true>), grid, block, 0, stream, a);
  } else if (rev) {
    launch_kernel((lpv_mimo_kernel<Alg, true>), grid, block, 0, stream, a);
  } else {
    launch_kernel((lpv_mimo_kernel<Alg, false>), grid, block, 0, stream, a);
  }
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

size_t phs_lpv_mimo_ss_workspace_size(int dtype, int M, int64_t B, int64_t T) {
  if (B < 0 || T < 0) return 0;
  size_t out = 0;
  const int rc = phs::mimo_dispatch(dtype, M, [&](auto alg) {
    out = phs::lpv_mimo_ws_bytes<decltype(alg)>(B, T);
    return PHS_OK;
  });
  return rc == PHS_OK ? out : 0;
}

int phs_lpv_mimo_ss(int dtype, int M, int F, int P, int64_t B, int64_t T, const void *A, int A_flags,
                    const void *Bm, const void *Cm, const void *Dm, int shared, const void *zi, const void *x,
                    void *y, void *zf, int reverse, void *workspace, size_t workspace_bytes, void *stream) {
  return phs_lpv_mimo_ss_hs(dtype, M, F, P, B, T, A, A_flags, Bm, Cm, Dm, shared, zi, x, y, zf, nullptr, reverse,
                            workspace, workspace_bytes, stream);
}

int phs_lpv_mimo_ss_hs(int dtype, int M, int F, int P, int64_t B, int64_t T, const void *A, int A_flags,
                       const void *Bm, const void *Cm, const void *Dm, int shared, const void *zi, const void *x,
                       void *y, void *zf, void *hs, int reverse, void *workspace, size_t workspace_bytes,
                       void *stream) {
  const hipStream_t st = static_cast<hipStream_t>(stream);
  return phs::mimo_dispatch(dtype, M, [&](auto alg) {
    return phs::lpv_mimo_ss<decltype(alg)>(F, P, B, T, A, A_flags, Bm, Cm, Dm, shared, zi, x, y, zf, workspace,
                                           workspace_bytes, reverse != 0, st, hs);
  });
}

size_t phs_mimo_ss_grad_sums_scratch_size(int dtype, int64_t B, int64_t T) {
  if (B < 0 || T < 0 || (dtype != PHS_F32 && dtype != PHS_F64)) return 0;
  const int64_t chunk = int64_t(phs::kSumThreads) * phs::kSumSteps;
  // the partials of every (row, block), then one total per row
  return size_t(B) * size_t((T + chunk - 1) / chunk + 1) * phs::kSumN * sizeof(double);
}

int phs_mimo_ss_grad_sums(int dtype, int M, int F, int P, int64_t B, int64_t T, const void *lam, const void *hs,
                          const void *x, const void *g, const void *Bm, const void *Dm, int shared, void *gA,
                          void *gB, void *gC, void *gD, void *gx, void *scratch, size_t scratch_bytes, void *stream) {
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == PHS_F32)
    return phs::grad_sums<float>(M, F, P, B, T, lam, hs, x, g, Bm, Dm, shared, gA, gB, gC, gD, gx, scratch,
                                 scratch_bytes, st);
  if (dtype == PHS_F64)
    return phs::grad_sums<double>(M, F, P, B, T, lam, hs, x, g, Bm, Dm, shared, gA, gB, gC, gD, gx, scratch,
                                  scratch_bytes, st);
  return PHS_ERR_DTYPE;
}

}  // extern "C"
