// C ABI of the fused second-order-section cascade (declared in
// include/philscan.h): argument checks, workspace carving and the launches of
// sos_kernel [-> sos_grad_reduce_kernel] on the caller's stream.  No
// allocation and no synchronisation.
// Workspace layout: [0, 2048) claim header, then the status words of every
// (row, section, tile), then (gradient backward only) per-tile, per-wave
// coefficient sums.
#include "phs_launch.hpp"
#include "phs_sos.hpp"

#include <algorithm>
#include <tuple>
#include <type_traits>

namespace phs {
namespace {

// Forward tiles: fp32 16 steps per lane in two rounds (against four rounds
// and 8- or 32-step lanes, measured with 3 data waves), fp64 8 steps in four
// rounds; a lane's rounds are independent chains and run interleaved.  The
// forward holds few registers (fp32 128: four waves per SIMD), so its
// workgroups are wide, 15 data waves (fp32; fp64 7) beside the look-back
// wave: a CU's wave slots hold one tile, 15/16 of them signal, and C4's call
// is 256 tiles of 30720 steps, all resident at once.  With 3 data waves it
// was 1264 tiles on 1024 resident slots, two generations: 92.3 -> 77.0 us.
// The gradient backward keeps four
// arrays of a lane's steps live and an LDS table of lane states per lane and
// round: fp32 takes 32 steps in one round (236 VGPRs, no spills; 4% faster
// at C4 than 16 steps in two rounds, which cost a second table entry and a
// second round of multipliers), fp64 8 steps in one round.
template <typename E>
using SosFwd = std::conditional_t<sizeof(E) == 4, SosShape<E, 16, 2, 15>, SosShape<E, 8, 4, 7>>;
template <typename E>
using SosBwd = std::conditional_t<sizeof(E) == 4, SosShape<E, 32, 1, 3>, SosShape<E, 8, 1, 3>>;

struct SosLayout {
  int64_t tiles_per_row = 0;
  size_t status_off = 0, partials_off = 0, total = 0;
};

template <typename E, class Sh>
SosLayout sos_layout(int64_t B, int64_t T, int S, bool grad) {
  SosLayout L;
  L.tiles_per_row = (T + Sh::kTile - 1) / Sh::kTile;
  L.status_off = align_up(kHeaderBytes);
  const size_t words = size_t(B) * size_t(S) * size_t(L.tiles_per_row) * kSosStatusWords;
  size_t off = align_up(L.status_off + words * sizeof(uint64_t));
  if (grad) {
    L.partials_off = off;
    off = align_up(off + size_t(B) * size_t(S) * size_t(L.tiles_per_row) * Sh::kWaves * 5 *
                             sizeof(typename Wide<E>::type));
  }
  L.total = off;
  return L;
}

template <typename E>
int64_t n_ckpt(int64_t T) {
  return (T + kSosCkptEvery<E> - 1) / kSosCkptEvery<E>;
}
inline int64_t n_ckpt_of(int dtype, int64_t T) { return dtype == PHS_F32 ? n_ckpt<float>(T) : n_ckpt<double>(T); }
inline int ckpt_every_of(int dtype) { return dtype == PHS_F32 ? kSosCkptEvery<float> : kSosCkptEvery<double>; }

template <typename E>
size_t ws_bytes_for(int64_t B, int64_t T, int S, bool backward) {
  size_t f = sos_layout<E, SosFwd<E>>(B, T, S, false).total;
  // one section: the biquad forward runs the state-space kernel
  if (S == 1) f = std::max(f, biquad_ss_ws_bytes(std::is_same<E, float>::value ? PHS_F32 : PHS_F64, B, T));
  if (!backward) return f;
  return std::max(f, sos_layout<E, SosBwd<E>>(B, T, S, true).total);
}

bool sizes_ok(int64_t B, int64_t T, int S) { return B >= 0 && T >= 0 && S >= 1 && S <= kSosMaxSections; }

// Dynamic LDS a launch of `kernel` may take on the current device with
// `wgs` of its workgroups resident per CU: the device's LDS per CU over wgs,
// at most its LDS per workgroup, less the kernel's static LDS (cached per
// kernel, device and wgs; 64 KiB per CU and per workgroup where the queries
// fail).
size_t lds_limit(const void *kernel, int wgs) {
  static std::mutex mu;
  static std::map<std::tuple<const void *, int, int>, size_t> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_tuple(kernel, dev, wgs);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int per_block = 0, per_cu = 0;
  hipFuncAttributes attr{};
  size_t stat = 0;
  if (hipFuncGetAttributes(&attr, kernel) == hipSuccess) stat = attr.sharedSizeBytes;
  if (dev < 0 || hipDeviceGetAttribute(&per_block, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
      per_block <= 0)
    per_block = 64 << 10;
  if (dev < 0 ||
      hipDeviceGetAttribute(&per_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess ||
      per_cu <= 0)
    per_cu = 64 << 10;
  const size_t avail = std::min(size_t(per_block), size_t(per_cu) / size_t(wgs > 0 ? wgs : 1));
  const size_t out = avail > stat ? avail - stat : 0;
  cache[key] = out;
  return out;
}

// Where the coefficients lie: a [rows, S, 6] sos array (shared: one row
// for all), or one biquad as lfilter's b [rows, nb] and a [rows, 2] at their
// own row strides (0 = shared).
struct SosCoefs {
  const void *sos = nullptr;
  bool shared = false;
  const void *b = nullptr, *a = nullptr;
  int64_t b_row_stride = 0, a_row_stride = 0;
  int nb = 0;
  bool coef_shared() const { return b ? (b_row_stride == 0 && a_row_stride == 0) : shared; }
  bool ok() const { return b ? (a && nb >= 1 && nb <= 3 && b_row_stride >= 0 && a_row_stride >= 0) : sos != nullptr; }
};

template <typename E, class Sh>
void fill_common(SosArgs<E> &a, const SosLayout &L, int64_t B, int64_t T, int S, const SosCoefs &k, char *ws) {
  a.sos = static_cast<const E *>(k.sos);
  a.sos_row_stride = k.shared ? 0 : int64_t(S) * 6;
  a.fb = static_cast<const E *>(k.b);
  a.fa = static_cast<const E *>(k.a);
  a.fb_row_stride = k.b_row_stride;
  a.fa_row_stride = k.a_row_stride;
  a.nb = k.nb;
  a.B = B;
  a.T_len = T;
  a.tiles_per_row = L.tiles_per_row;
  a.n_ckpt = n_ckpt<E>(T);
  a.S = S;
  a.claims = reinterpret_cast<unsigned long long *>(ws);
  a.status = reinterpret_cast<uint64_t *>(ws + L.status_off);
  a.tiles = unsigned(B * L.tiles_per_row);
  row_split(B, a.b_magic, a.b_shift);
  a.per_stripe = (a.tiles + kStripes - 1) / kStripes;
  const unsigned sl = g_spin_limit.load(std::memory_order_relaxed);
  a.spin_limit = sl ? sl : kDefaultSpinLimit;
  a.agg_only = g_agg_only.load(std::memory_order_relaxed) ? 1u : 0u;
}

template <typename E>
int sos_fwd(int64_t B, int64_t T, int S, const SosCoefs &k, const void *zi, const void *x, void *y, void *zf,
            void *ckpt, void *workspace, size_t ws_bytes, hipStream_t stream) {
  using Sh = SosFwd<E>;
  if (!sizes_ok(B, T, S) || (k.b && S != 1)) return PHS_ERR_INVALID;
  if (B == 0 || T == 0) return PHS_OK;
  if (!k.ok() || !x || !y) return PHS_ERR_INVALID;
  const SosLayout L = sos_layout<E, Sh>(B, T, S, false);
  if (double(B) * double(L.tiles_per_row) >= 2147483648.0) return PHS_ERR_INVALID;
  if (!workspace || ws_bytes < L.total) return PHS_ERR_WORKSPACE;
  SosArgs<E> a{};
  fill_common<E, Sh>(a, L, B, T, S, k, static_cast<char *>(workspace));
  a.in = static_cast<const E *>(x);
  a.out = static_cast<E *>(y);
  a.virt = static_cast<const E *>(zi);
  a.fin = static_cast<E *>(zf);
  a.ckpt = static_cast<Vec2<typename Wide<E>::type> *>(ckpt);
  a.vec_ok = (size_t(T) * sizeof(E)) % 16 == 0 && aligned16(x) && aligned16(y);
  const unsigned grid = a.per_stripe * kStripes;
  launch_kernel((sos_kernel<E, Sh, false, false>), dim3(grid), dim3(Sh::kThreads), 0, stream, a);
  return hipGetLastError() == hipSuccess ? PHS_OK : PHS_ERR_LAUNCH;
}

// gsos (sos layout) or gb, ga (biquad layout): the coefficient gradients,
// null for none.
template <typename E>
int sos_bwd(int64_t B, int64_t T, int S, const SosCoefs &k, const void *x, const void *ckpt, const void *gy,
            const void *gzf, void *gx, void *gsos, void *gb, void *ga, void *gzi, void *workspace, size_t ws_bytes,
            hipStream_t stream, int b_cols = 1, int b_col = 0, int a_cols = 1, int a_col = 0) {
  using Sh = SosBwd<E>;
  if (!sizes_ok(B, T, S) || (k.b && S != 1)) return PHS_ERR_INVALID;
  if (B == 0 || T == 0) return PHS_OK;
  if (k.b ? (gsos != nullptr || (gb == nullptr) != (ga == nullptr)) : (gb || ga)) return PHS_ERR_INVALID;
  const bool grad = k.b ? gb != nullptr : gsos != nullptr;
  if (!k.ok() || !gy || (grad && (!x || !ckpt))) return PHS_ERR_INVALID;
  const SosLayout L = sos_layout<E, Sh>(B, T, S, grad);
  if (double(B) * double(L.tiles_per_row) >= 2147483648.0) return PHS_ERR_INVALID;
  if (!workspace || ws_bytes < L.total) return PHS_ERR_WORKSPACE;
  char *ws = static_cast<char *>(workspace);
  SosArgs<E> a{};
  fill_common<E, Sh>(a, L, B, T, S, k, ws);
  a.in = static_cast<const E *>(gy);
  a.out = static_cast<E *>(gx);
  a.virt = static_cast<const E *>(gzf);
  a.fin = static_cast<E *>(gzi);
  a.ckpt = const_cast<Vec2<typename Wide<E>::type> *>(static_cast<const Vec2<typename Wide<E>::type> *>(ckpt));
  a.x = static_cast<const E *>(x);
  a.partials = grad ? reinterpret_cast<typename Wide<E>::type *>(ws + L.partials_off) : nullptr;
  a.vec_ok = (size_t(T) * sizeof(E)) % 16 == 0 && aligned16(gy) && aligned16(gx) && (!grad || aligned16(x));
  const unsigned grid = a.per_stripe * kStripes;
  if (grad) {
    // lane entry states of every section, then the kept sections' inputs:
    // every third section where the LDS left to each of the workgroups the
    // kernel's registers let a CU hold allows two slots, else every other
    // (fp32 on gfx950: three workgroups per CU, one slot), else none
    const size_t laneh = size_t(S) * Sh::kWaves * Sh::R * 64 * sizeof(Vec2<E>);
    const size_t slot = size_t(Sh::kWaves) * Sh::R * Sh::K * 64 * sizeof(E);
    // one section with room for the output's slot: the form that parks x
    // there (ONE in sos_kernel)
    const auto kernel_one = sos_kernel<E, Sh, true, true, true>;
    const bool one = S == 1 && laneh + slot <= lds_limit(reinterpret_cast<const void *>(kernel_one),
                                                         kSosWgsPerCu<E, Sh, true>);
    const auto kernel = one ? kernel_one : sos_kernel<E, Sh, true, true>;
    const size_t limit = lds_limit(reinterpret_cast<const void *>(kernel), kSosWgsPerCu<E, Sh, true>);
    int step = S >= 2 ? (S + 2) / 3 : 0;
    if (step > 0 && laneh + sos_kept_slots(S, step) * slot > limit) step = (S + 1) / 2;
    if (step > 0 && laneh + sos_kept_slots(S, step) * slot > limit) step = 0;
    const int forced = g_sos_kept_step.load(std::memory_order_relaxed);  // testing hook
    if (forced >= 0) {
      if (laneh + sos_kept_slots(S, forced) * slot > limit) return PHS_ERR_INVALID;
      step = forced;
    }
    a.kept_step = step;
    size_t lds = laneh + sos_kept_slots(S, step) * slot;
    // kept slot 0 also takes the output's LDS transpose at the end; without
    // kept inputs, one slot is added for it where the LDS allows
    a.out_lds = 0;
    if (sos_kept_slots(S, step) >= 1) {
      a.out_lds = 1;
    } else if (laneh + slot <= limit) {
      lds = laneh + slot;
      a.out_lds = 1;
    }
    launch_kernel(kernel, dim3(grid), dim3(Sh::kThreads), lds, stream, a);
    if (hipGetLastError() != hipSuccess) return PHS_ERR_LAUNCH;
    const int64_t rows = k.coef_shared() ? 1 : B;
    hipLaunchKernelGGL((sos_grad_reduce_kernel<E, Sh>), dim3(unsigned(rows * S)), dim3(kSosReduceThreads), 0,
                       stream, a, static_cast<E *>(gsos), rows, static_cast<E *>(gb), static_cast<E *>(ga), b_cols,
                       b_col, a_cols, a_col);
  } else {
    launch_kernel((sos_kernel<E, Sh, true, false>), dim3(grid), dim3(Sh::kThreads), 0, stream, a);
  }
  return hipGetLastError() == hipSuccess ? PHS_OK : PHS_ERR_LAUNCH;
}

}  // namespace
}  // namespace phs

extern "C" {

size_t phs_sosfilt_workspace_size(int dtype, int64_t B, int64_t T, int S, int backward) {
  if (!phs::sizes_ok(B, T, S)) return 0;
  switch (dtype) {
    case PHS_F32: return phs::ws_bytes_for<float>(B, T, S, backward != 0);
    case PHS_F64: return phs::ws_bytes_for<double>(B, T, S, backward != 0);
    default: return 0;
  }
}

size_t phs_sosfilt_ckpt_size(int dtype, int64_t B, int64_t T, int S) {
  if (!phs::sizes_ok(B, T, S) || (dtype != PHS_F32 && dtype != PHS_F64)) return 0;
  return size_t(B) * size_t(S) * size_t(phs::n_ckpt_of(dtype, T)) * 2 * sizeof(double);
}

int phs_sosfilt_fwd(int dtype, int64_t B, int64_t T, int S, const void *sos, int sos_shared, const void *zi,
                    const void *x, void *y, void *zf, void *ckpt, void *workspace, size_t workspace_bytes,
                    void *stream) {
  const hipStream_t st = static_cast<hipStream_t>(stream);
  phs::SosCoefs k;
  k.sos = sos;
  k.shared = sos_shared != 0;
  switch (dtype) {
    case PHS_F32: return phs::sos_fwd<float>(B, T, S, k, zi, x, y, zf, ckpt, workspace, workspace_bytes, st);
    case PHS_F64: return phs::sos_fwd<double>(B, T, S, k, zi, x, y, zf, ckpt, workspace, workspace_bytes, st);
    default: return PHS_ERR_DTYPE;
  }
}

int phs_sosfilt_bwd(int dtype, int64_t B, int64_t T, int S, const void *sos, int sos_shared, const void *x,
                    const void *ckpt, const void *grad_y, const void *grad_zf, void *grad_x, void *grad_sos,
                    void *grad_zi, void *workspace, size_t workspace_bytes, void *stream) {
  const hipStream_t st = static_cast<hipStream_t>(stream);
  phs::SosCoefs k;
  k.sos = sos;
  k.shared = sos_shared != 0;
  switch (dtype) {
    case PHS_F32:
      return phs::sos_bwd<float>(B, T, S, k, x, ckpt, grad_y, grad_zf, grad_x, grad_sos, nullptr, nullptr, grad_zi,
                                 workspace, workspace_bytes, st);
    case PHS_F64:
      return phs::sos_bwd<double>(B, T, S, k, x, ckpt, grad_y, grad_zf, grad_x, grad_sos, nullptr, nullptr, grad_zi,
                                  workspace, workspace_bytes, st);
    default: return PHS_ERR_DTYPE;
  }
}

namespace {
phs::SosCoefs biquad_coefs(const void *b, int nb, int64_t b_row_stride, const void *a, int64_t a_row_stride) {
  phs::SosCoefs k;
  k.b = b;
  k.a = a;
  k.nb = nb;
  k.b_row_stride = b_row_stride;
  k.a_row_stride = a_row_stride;
  return k;
}
}  // namespace

int phs_biquad_fwd(int dtype, int64_t B, int64_t T, const void *b, int nb, int64_t b_row_stride, const void *a,
                   int64_t a_row_stride, const void *zi, const void *x, void *y, void *zf, void *ckpt,
                   void *workspace, size_t workspace_bytes, void *stream) {
  // the plain state-space pass of the TDF-II model (shorter than the
  // cascade kernel at one section), writing the cascade's checkpoints for
  // phs_biquad_bwd
  if (dtype != PHS_F32 && dtype != PHS_F64) return PHS_ERR_DTYPE;
  if (nb < 1 || nb > 3) return PHS_ERR_INVALID;
  return phs::biquad_fwd_ss(dtype, B, T, b, nb, b_row_stride, a, a_row_stride, zi, x, y, zf, ckpt,
                            phs::n_ckpt_of(dtype, T), phs::ckpt_every_of(dtype), workspace, workspace_bytes,
                            static_cast<hipStream_t>(stream));
}

int phs_biquad_bwd_cols(int dtype, int64_t B, int64_t T, const void *b, int nb, int64_t b_row_stride, const void *a,
                        int64_t a_row_stride, const void *x, const void *ckpt, const void *grad_y,
                        const void *grad_zf, void *grad_x, void *grad_b_table, int b_cols, int b_col,
                        void *grad_a_table, int a_cols, int a_col, void *grad_zi, void *workspace,
                        size_t workspace_bytes, void *stream) {
  if (b_cols < 1 || b_col < 0 || b_col >= b_cols || a_cols < 1 || a_col < 0 || a_col >= a_cols)
    return PHS_ERR_INVALID;
  if ((grad_b_table == nullptr) != (grad_a_table == nullptr)) return PHS_ERR_INVALID;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const phs::SosCoefs k = biquad_coefs(b, nb, b_row_stride, a, a_row_stride);
  switch (dtype) {
    case PHS_F32:
      return phs::sos_bwd<float>(B, T, 1, k, x, ckpt, grad_y, grad_zf, grad_x, nullptr, grad_b_table, grad_a_table,
                                 grad_zi, workspace, workspace_bytes, st, b_cols, b_col, a_cols, a_col);
    case PHS_F64:
      return phs::sos_bwd<double>(B, T, 1, k, x, ckpt, grad_y, grad_zf, grad_x, nullptr, grad_b_table, grad_a_table,
                                  grad_zi, workspace, workspace_bytes, st, b_cols, b_col, a_cols, a_col);
    default: return PHS_ERR_DTYPE;
  }
}

int phs_biquad_bwd(int dtype, int64_t B, int64_t T, const void *b, int nb, int64_t b_row_stride, const void *a,
                   int64_t a_row_stride, const void *x, const void *ckpt, const void *grad_y, const void *grad_zf,
                   void *grad_x, void *grad_b, void *grad_a, void *grad_zi, void *workspace, size_t workspace_bytes,
                   void *stream) {
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const phs::SosCoefs k = biquad_coefs(b, nb, b_row_stride, a, a_row_stride);
  switch (dtype) {
    case PHS_F32:
      return phs::sos_bwd<float>(B, T, 1, k, x, ckpt, grad_y, grad_zf, grad_x, nullptr, grad_b, grad_a, grad_zi,
                                 workspace, workspace_bytes, st);
    case PHS_F64:
      return phs::sos_bwd<double>(B, T, 1, k, x, ckpt, grad_y, grad_zf, grad_x, nullptr, grad_b, grad_a, grad_zi,
                                  workspace, workspace_bytes, st);
    default: return PHS_ERR_DTYPE;
  }
}

}  // extern "C"
