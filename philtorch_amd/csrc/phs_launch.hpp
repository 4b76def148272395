// Host side shared by the C ABI units (phs_capi.hip: fixed-order entry points;
// phs_capi_n.hip: order-M entry points): argument checks, workspace carving,
// and the launch of scan_kernel [-> reduce kernel] on the caller's stream.
// No allocation and no synchronisation; the only global state is the
// testing and measurement hooks and a per-device cache of how many
// workgroups of each kernel are resident at once.
// Workspace layout: [0, 2048) header (16 striped {epoch, claim count} words),
// then the tile status words, then (backward only) per-tile partial sums or
// per-step scratch.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <utility>

#include "../../include/philscan.h"
#include "phs_scan.hpp"

namespace phs {

inline constexpr size_t kAlign = 256;
// Look-back polls before a tile computes its entry state itself; about 0.1 s
// of waiting, far beyond any schedule in which predecessors make progress.
inline constexpr unsigned kDefaultSpinLimit = 1u << 16;
extern std::atomic<unsigned> g_spin_limit;  // testing hook, 0 = default (phs_capi.hip)
extern std::atomic<bool> g_agg_only;        // testing hook (phs_capi.hip)
extern std::atomic<int> g_sos_kept_step;    // testing hook, < 0 = automatic (phs_capi.hip)
inline size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// Measurement hook (phs_debug_time_next_launch): a pair of events that the
// next main-kernel launch of the library records around the kernel itself
// (hipExtLaunchKernelGGL), so their elapsed time is that kernel's own
// duration, dispatch to completion, with no event packets in between.  Taken
// (and cleared) by that launch.
struct TimingHook {
  std::atomic<bool> armed{false};
  std::mutex mu;
  hipEvent_t start = nullptr, stop = nullptr;
};
extern TimingHook g_timing;  // phs_capi.hip

inline bool take_timing(hipEvent_t &start, hipEvent_t &stop) {
  if (!g_timing.armed.load(std::memory_order_acquire)) return false;
  std::lock_guard<std::mutex> lock(g_timing.mu);
  if (!g_timing.armed.load(std::memory_order_relaxed)) return false;
  start = g_timing.start;
  stop = g_timing.stop;
  g_timing.armed.store(false, std::memory_order_relaxed);
  return true;
}

// Measurement hook (phs_debug_trace_next_launch): a device buffer of
// per-tile phase records that the next scan_kernel launch of a traceable
// algebra (TraceableAlg) fills, if its tiles fit.  Taken (and cleared) by
// that launch.
struct TraceHook {
  std::atomic<bool> armed{false};
  std::mutex mu;
  uint64_t *records = nullptr;
  size_t n_records = 0;
};
extern TraceHook g_trace;  // phs_capi.hip

// The algebras whose scans carry a tracing instantiation: those of the
// benchmark configurations (fp32/fp64 scalar, complex64 scalar, fp32 2x2).
template <class Alg>
struct TraceableAlg : std::false_type {};
template <>
struct TraceableAlg<Scalar<float>> : std::true_type {};
template <>
struct TraceableAlg<Scalar<double>> : std::true_type {};
template <>
struct TraceableAlg<Scalar<c64>> : std::true_type {};
template <>
struct TraceableAlg<Block2<float>> : std::true_type {};

inline bool take_trace(uint64_t *&records, size_t &n) {
  if (!g_trace.armed.load(std::memory_order_acquire)) return false;
  std::lock_guard<std::mutex> lock(g_trace.mu);
  if (!g_trace.armed.load(std::memory_order_relaxed)) return false;
  records = g_trace.records;
  n = g_trace.n_records;
  g_trace.armed.store(false, std::memory_order_relaxed);
  return true;
}

// Launch of a library kernel on `stream`, timed when the hook is armed.
template <typename F, typename... Args>
void launch_kernel(F kernel, dim3 grid, dim3 block, unsigned lds, hipStream_t stream, Args... args) {
  hipEvent_t start = nullptr, stop = nullptr;
  if (take_timing(start, stop))
    hipExtLaunchKernelGGL(kernel, grid, block, lds, stream, start, stop, 0u, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
}

struct Layout {
  int64_t tiles_per_row = 0;
  size_t status_off = 0, status_words = 0;  // header lives at offset 0
  size_t partials_off = 0, scratch_off = 0, total = 0;
};

// TV: coefficient varies with time; shared: one coefficient set for all rows.
template <class Alg>
Layout make_layout(int64_t B, int64_t T, bool TV, bool shared, bool backward) {
  const int64_t tile = TV ? Shape<Alg, true>::kTile : Shape<Alg, false>::kTile;
  Layout L;
  L.tiles_per_row = (T + tile - 1) / tile;
  L.status_off = align_up(kHeaderBytes);
  L.status_words = size_t(B) * size_t(L.tiles_per_row) * StatusShape<Alg>::kStride;
  size_t off = align_up(L.status_off + L.status_words * sizeof(uint64_t));
  if (backward && !TV) {  // per-tile coefficient-gradient partial sums
    L.partials_off = off;
    off = align_up(off + size_t(B) * size_t(L.tiles_per_row) * sizeof(typename Alg::acc_coef));
  }
  if (backward && TV && shared) {  // per-step gradients before the batch sum
    L.scratch_off = off;
    off = align_up(off + size_t(B) * size_t(T) * sizeof(typename Alg::s_coef));
  }
  L.total = off;
  return L;
}

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Tile id -> row by multiply and shift (the kernels' `id / B` without a
// 64-bit division): with l = ceil(log2 B) and s = 31 + l, m = floor(2^s / B)
// + 1 gives floor(id m / 2^s) = floor(id / B) for every id below 2^31
// (m B - 2^s lies in (0, B], and B <= 2^l).
inline void row_split(int64_t B, uint64_t &magic, unsigned &shift) {
  unsigned l = 0;
  while ((uint64_t(1) << l) < uint64_t(B)) ++l;
  shift = 31u + l;
  magic = ((uint64_t(1) << shift) / uint64_t(B)) + 1u;
}

// Workgroups of `kernel` resident at once on the current device (occupancy
// per CU times CUs), cached per (kernel, device); 0 if the query fails.
inline int64_t resident_groups(const void *kernel, int threads) {
  static std::mutex mu;
  static std::map<std::pair<const void *, int>, int64_t> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_pair(kernel, dev);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  const int64_t n = int64_t(std::max(per_cu, 0)) * std::max(cus, 0);
  cache[key] = n;
  return n;
}

template <class Alg, bool TV, bool REV>
void launch_scan(ScanArgs<Alg> a, unsigned grid, hipStream_t stream) {
  if constexpr (TraceableAlg<Alg>::value) {
    uint64_t *records = nullptr;
    size_t n = 0;
    if (take_trace(records, n) && records && n >= a.tiles) {
      a.trace = records;
      a.trace_tiles = a.tiles;
      launch_kernel(scan_kernel<Alg, TV, REV, true>, dim3(grid), dim3(Shape<Alg, TV>::kThreads), 0, stream, a);
      return;
    }
  }
  launch_kernel(scan_kernel<Alg, TV, REV>, dim3(grid), dim3(Shape<Alg, TV>::kThreads), 0, stream, a);
}

template <class Alg>
int launch(int64_t B, int64_t T, bool TV, bool shared, bool backward, const void *coef,
           const void *zi, const void *x, const void *y, void *out, void *gcoef, void *gzi,
           void *workspace, size_t ws_bytes, hipStream_t stream) {
  using E = typename Alg::elem;
  if (B < 0 || T < 0) return PHS_ERR_INVALID;
  if (B == 0 || T == 0) return PHS_OK;
  if (!coef || !zi || !x || (backward ? !y : !out)) return PHS_ERR_INVALID;
  const Layout L = make_layout<Alg>(B, T, TV, shared, backward);
  if (double(B) * double(L.tiles_per_row) >= 2147483648.0) return PHS_ERR_INVALID;
  if (!workspace || ws_bytes < L.total) return PHS_ERR_WORKSPACE;

  char *ws = static_cast<char *>(workspace);
  ScanArgs<Alg> a{};
  a.coef = static_cast<const E *>(coef);
  a.coef_row_stride = shared ? 0 : (TV ? T : 1);
  a.zi = static_cast<const E *>(zi);
  a.x = static_cast<const E *>(x);
  a.y = static_cast<const E *>(y);
  a.out = static_cast<E *>(out);
  a.gcoef = nullptr;
  a.partials = nullptr;
  a.gzi = static_cast<E *>(gzi);
  a.B = B;
  a.T_len = T;
  a.tiles_per_row = L.tiles_per_row;
  a.claims = reinterpret_cast<unsigned long long *>(ws);
  a.status = reinterpret_cast<uint64_t *>(ws + L.status_off);
  const unsigned tiles = unsigned(B * L.tiles_per_row);
  a.tiles = tiles;
  a.per_stripe = (tiles + kStripes - 1) / kStripes;
  const unsigned sl = g_spin_limit.load(std::memory_order_relaxed);
  a.spin_limit = sl ? sl : kDefaultSpinLimit;
  a.agg_only = g_agg_only.load(std::memory_order_relaxed) ? 1u : 0u;
  row_split(B, a.b_magic, a.b_shift);
  a.trace = nullptr;
  a.trace_tiles = 0;
  if (backward && gcoef) {
    if (TV)
      a.gcoef = shared ? reinterpret_cast<E *>(ws + L.scratch_off) : static_cast<E *>(gcoef);
    else
      a.partials = ws + L.partials_off;
  }
  bool vec = (size_t(T) * sizeof(typename Alg::s_state)) % 16 == 0 && aligned16(x) && aligned16(y) &&
             aligned16(out) && aligned16(a.gcoef) && (!TV || aligned16(coef));
  a.vec_ok = vec ? 1 : 0;

  const void *kernel = TV ? (backward ? reinterpret_cast<const void *>(scan_kernel<Alg, true, true>)
                                       : reinterpret_cast<const void *>(scan_kernel<Alg, true, false>))
                          : (backward ? reinterpret_cast<const void *>(scan_kernel<Alg, false, true>)
                                      : reinterpret_cast<const void *>(scan_kernel<Alg, false, false>));
  // Tiles are claimed q-major, so a tile's predecessor in its row was claimed
  // B claims earlier, i.e. B/resident tile lifetimes earlier.  From half a
  // lifetime on it has published at least its aggregate, and the look-back
  // wave can poll for it while the data waves are still loading; with
  // smaller B those early polls mostly fail and only add status traffic.
  a.early_polls = 0;
  if (Alg::kLookbackWave && !a.agg_only) {
    const int threads = TV ? Shape<Alg, true>::kThreads : Shape<Alg, false>::kThreads;
    const int64_t resident = resident_groups(kernel, threads);
    if (resident > 0 && 2 * B >= resident) a.early_polls = a.spin_limit;
  }

  const unsigned grid = a.per_stripe * kStripes;
  if (TV) {
    if (backward)
      launch_scan<Alg, true, true>(a, grid, stream);
    else
      launch_scan<Alg, true, false>(a, grid, stream);
  } else {
    if (backward)
      launch_scan<Alg, false, true>(a, grid, stream);
    else
      launch_scan<Alg, false, false>(a, grid, stream);
  }
  if (backward && gcoef) {
    if (TV && shared) {
      const int blocks = int(std::min<int64_t>((T + kReduceThreads - 1) / kReduceThreads, 4096));
      hipLaunchKernelGGL(reduce_batch_kernel<Alg>, dim3(blocks), dim3(kReduceThreads), 0, stream,
                         static_cast<const E *>(a.gcoef), B, T, static_cast<E *>(gcoef));
    } else if (!TV) {
      const int64_t rows = shared ? 1 : B;
      const int64_t count = shared ? B * L.tiles_per_row : L.tiles_per_row;
      hipLaunchKernelGGL(reduce_rows_kernel<Alg>, dim3(unsigned(rows)), dim3(kReduceThreads), 0, stream,
                         static_cast<const void *>(a.partials), count, static_cast<E *>(gcoef));
    }
  }
  return hipGetLastError() == hipSuccess ? PHS_OK : PHS_ERR_LAUNCH;
}

template <template <class> class AlgT, class F>
int dispatch(int dtype, F &&f) {
  switch (dtype) {
    case PHS_F32: return f(AlgT<float>{});
    case PHS_F64: return f(AlgT<double>{});
    case PHS_C64: return f(AlgT<c64>{});
    case PHS_C128: return f(AlgT<c128>{});
    case PHS_I64: return f(AlgT<int64_t>{});
    default: return PHS_ERR_DTYPE;
  }
}

template <template <class> class AlgT>
size_t ws_size(int dtype, int64_t B, int64_t T, bool TV, bool shared, bool backward) {
  size_t out = 0;
  if (B <= 0 || T <= 0) return 0;
  dispatch<AlgT>(dtype, [&](auto alg) {
    using Alg = decltype(alg);
    out = make_layout<Alg>(B, T, TV, shared, backward).total;
    return 0;
  });
  return out;
}

// Order-M (3, 4) launches and workspace sizes of the generic BlockN
// algebra.  Declared here, defined in phs_blockn.hip, which is compiled once
// per order (its instantiations are the costly ones to build).
template <int M>
int launch_blockn(int dtype, int64_t B, int64_t T, bool TV, bool shared, bool backward, const void *coef,
                  const void *zi, const void *x, const void *y, void *out, void *gcoef, void *gzi,
                  void *workspace, size_t ws_bytes, hipStream_t stream);
template <int M>
size_t ws_blockn(int dtype, int64_t B, int64_t T, bool TV, bool shared, bool backward);

// One biquad's forward on the state-space kernel with the fused cascade's
// checkpoints, and its workspace bytes (defined in phs_ss.hip; the biquad
// entry points live in phs_sos.hip).
int biquad_fwd_ss(int dtype, int64_t B, int64_t T, const void *b, int nb, int64_t b_row_stride, const void *a,
                  int64_t a_row_stride, const void *zi, const void *x, void *y, void *zf, void *ckpt, int64_t n_ckpt,
                  int ckpt_every, void *workspace, size_t ws_bytes, hipStream_t stream);
size_t biquad_ss_ws_bytes(int dtype, int64_t B, int64_t T);

}  // namespace phs
