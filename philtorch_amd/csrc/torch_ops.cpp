// torch.library layer of philtorch_amd: owns the `philtorch` operator
// namespace with the reference's schemas (philtorch/csrc/host_recur2.cpp:162-171)
// plus the new LPV scalar op `recur`, four fused backward ops and the fused
// filter ops (`sosfilt`, `filtfilt`, `lti_ss`, `lfilter_ss`, `lpv_ss`, `mimo_ss`, `lpv_mimo_ss`), and
// binds the HIP device key (PyTorch-ROCm names it CUDA) to the C ABI of
// libphilscan.  The CPU key serves the reference's five ops, `recur` and the
// backward ops with the CPU kernels of phs_cpu.hpp, as the reference's CPU
// extension does for its ops (host_recurN.cpp:283-287, host_lti_recur.cpp:
// 82-85, host_lti_recurN.cpp:110-114); the filter ops are HIP-only (the
// Python API composes them from the basic ops on CPU tensors).
#include <ATen/ATen.h>
#include <ATen/Dispatch.h>
#include <ATen/Parallel.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <optional>
#include <tuple>
#include <vector>

#include "../../include/philscan.h"
#include "phs_cpu.hpp"

namespace {

using at::Tensor;
using Triple = std::tuple<Tensor, Tensor, Tensor>;

int phs_dtype_of(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return PHS_F32;
    case at::kDouble: return PHS_F64;
    case at::kComplexFloat: return PHS_C64;
    case at::kComplexDouble: return PHS_C128;
    case at::kLong: return PHS_I64;
    default: return -1;
  }
}

bool is_half(at::ScalarType t) { return t == at::kHalf || t == at::kBFloat16; }

void check_status(int rc, const char *op) {
  TORCH_CHECK(rc == PHS_OK, "philtorch::", op, ": ", phs_error_string(rc));
}

void check_common(const char *op, const Tensor &A, const Tensor &zi, const Tensor &x) {
  // message texts follow host_recurN.cpp:240-248 / host_lti_recur.cpp:45-50
  TORCH_CHECK(zi.scalar_type() == x.scalar_type(), "zi must have the same scalar type as input");
  TORCH_CHECK(A.scalar_type() == x.scalar_type(), "A must have the same scalar type as input");
  TORCH_CHECK(A.device() == x.device() && zi.device() == x.device(), "philtorch::", op,
              ": all tensors must be on the same device");
  TORCH_CHECK(is_half(x.scalar_type()) || phs_dtype_of(x.scalar_type()) >= 0, "philtorch::", op,
              ": unsupported dtype ", x.scalar_type());
}

void *stream_of(const Tensor &t) {
  return c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream();
}

// The kernels' workspace is self-resetting: zero-filled once, then every call
// leaves it ready for the next one on the same stream.  One buffer is kept per
// (device, stream) and grown geometrically; a replaced buffer goes back to the
// caching allocator, whose stream-ordered reuse keeps in-flight kernels safe.
// Status words carry a 32-bit per-call tag, so the buffer is zeroed again
// every 2^31 calls, long before a tag could repeat.
// The cache is intentionally leaked at exit (no HIP calls during teardown).
struct Workspace {
  void *ptr;
  size_t bytes;
};

struct CachedWorkspace {
  Tensor buf;
  uint64_t calls = 0;
};

Workspace workspace_for(const Tensor &like, size_t bytes, void *stream) {
  static auto *mu = new std::mutex;
  static auto *cache = new std::map<std::pair<int, void *>, CachedWorkspace>;
  std::lock_guard<std::mutex> lock(*mu);
  CachedWorkspace &entry = (*cache)[std::make_pair(int(like.device().index()), stream)];
  if (!entry.buf.defined() || size_t(entry.buf.numel()) < bytes) {
    size_t cap = size_t(1) << 16;
    if (entry.buf.defined()) cap = std::max(cap, size_t(entry.buf.numel()) * 2);
    while (cap < bytes) cap *= 2;
    entry.buf = at::zeros({int64_t(cap)}, like.options().dtype(at::kByte));
    entry.calls = 0;
  } else if (++entry.calls >= (uint64_t(1) << 31)) {
    entry.buf.zero_();
    entry.calls = 0;
  }
  return {entry.buf.mutable_data_ptr(), size_t(entry.buf.numel())};
}

// Largest state order with native kernels (the C ABI's phs_*N_* entry points).
constexpr int64_t kMaxOrder = 4;

using FwdFn = int (*)(int, int64_t, int64_t, const void *, int, const void *, const void *, void *,
                      void *, size_t, void *);
using BwdFn = int (*)(int, int64_t, int64_t, const void *, int, const void *, const void *,
                      const void *, void *, void *, void *, void *, size_t, void *);

// y = op(A, zi, x); A/zi/x already validated, x is [B, T, ...].
// launch(dt, B, T, A, shared, zi, x, y, ws, bytes, stream) runs the entry
// point; ws_size(dt, B, T, shared, backward) sizes its workspace.
template <class Launch, class Size>
Tensor run_fwd_with(const char *name, Launch &&launch, Size &&ws_size, const Tensor &A, bool shared,
                    const Tensor &zi, const Tensor &x) {
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  const int dt = phs_dtype_of(x.scalar_type());
  const int64_t B = x.size(0), T = x.size(1);
  Tensor Ac = A.contiguous(), zc = zi.contiguous(), xc = x.contiguous();
  Tensor y = at::empty_like(xc, at::MemoryFormat::Contiguous);
  void *stream = stream_of(x);
  const Workspace ws = workspace_for(x, ws_size(dt, B, T, shared ? 1 : 0, 0), stream);
  check_status(launch(dt, B, T, Ac.const_data_ptr(), shared ? 1 : 0, zc.const_data_ptr(), xc.const_data_ptr(),
                      y.mutable_data_ptr(), ws.ptr, ws.bytes, stream),
               name);
  return y;
}

template <class Launch, class Size>
Triple run_bwd_with(const char *name, Launch &&launch, Size &&ws_size, const Tensor &A, bool shared,
                    const Tensor &zi, const Tensor &y, const Tensor &gy) {
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(y.device());
  const int dt = phs_dtype_of(y.scalar_type());
  const int64_t B = y.size(0), T = y.size(1);
  Tensor Ac = A.contiguous(), zc = zi.contiguous(), yc = y.contiguous(), gc = gy.contiguous();
  Tensor gA = at::empty(A.sizes(), A.options());
  Tensor gzi = at::empty(zi.sizes(), zi.options());
  Tensor gx = at::empty(y.sizes(), y.options());
  void *stream = stream_of(y);
  const Workspace ws = workspace_for(y, ws_size(dt, B, T, shared ? 1 : 0, 1), stream);
  check_status(launch(dt, B, T, Ac.const_data_ptr(), shared ? 1 : 0, zc.const_data_ptr(), yc.const_data_ptr(),
                      gc.const_data_ptr(), gx.mutable_data_ptr(), gA.mutable_data_ptr(), gzi.mutable_data_ptr(),
                      ws.ptr, ws.bytes, stream),
               name);
  if (B == 0 || T == 0) {  // nothing was launched: gradients are zero
    gA.zero_();
    gzi.zero_();
    gx.zero_();
  }
  return {gA, gzi, gx};
}

// fixed-order entry points (op: a phs_op of order 1 or 2)
Tensor run_fwd(const char *name, FwdFn fn, int op, const Tensor &A, bool shared, const Tensor &zi,
               const Tensor &x) {
  return run_fwd_with(
      name, fn, [op](int dt, int64_t B, int64_t T, int sh, int bw) { return phs_workspace_size(op, dt, B, T, sh, bw); },
      A, shared, zi, x);
}

Triple run_bwd(const char *name, BwdFn fn, int op, const Tensor &A, bool shared, const Tensor &zi,
               const Tensor &y, const Tensor &gy) {
  return run_bwd_with(
      name, fn, [op](int dt, int64_t B, int64_t T, int sh, int bw) { return phs_workspace_size(op, dt, B, T, sh, bw); },
      A, shared, zi, y, gy);
}

// order-M entry points (phs_recurN_* / phs_lti_recurN_*, op PHS_OP_RECURN or
// PHS_OP_LTI_RECURN)
using FwdFnN = int (*)(int, int, int64_t, int64_t, const void *, int, const void *, const void *, void *,
                       void *, size_t, void *);
using BwdFnN = int (*)(int, int, int64_t, int64_t, const void *, int, const void *, const void *,
                       const void *, void *, void *, void *, void *, size_t, void *);

Tensor run_fwd_n(const char *name, FwdFnN fn, int op, int M, const Tensor &A, bool shared, const Tensor &zi,
                 const Tensor &x) {
  return run_fwd_with(
      name, [fn, M](int dt, auto... rest) { return fn(dt, M, rest...); },
      [op, M](int dt, int64_t B, int64_t T, int sh, int bw) { return phs_workspace_size_n(op, dt, M, B, T, sh, bw); },
      A, shared, zi, x);
}

Triple run_bwd_n(const char *name, BwdFnN fn, int op, int M, const Tensor &A, bool shared, const Tensor &zi,
                 const Tensor &y, const Tensor &gy) {
  return run_bwd_with(
      name, [fn, M](int dt, auto... rest) { return fn(dt, M, rest...); },
      [op, M](int dt, int64_t B, int64_t T, int sh, int bw) { return phs_workspace_size_n(op, dt, M, B, T, sh, bw); },
      A, shared, zi, y, gy);
}

Triple to_dtype(const Triple &t, at::ScalarType dt) {
  return {std::get<0>(t).to(dt), std::get<1>(t).to(dt), std::get<2>(t).to(dt)};
}

// ------------------------------------------------------------ LPV scalar
void check_recur(const Tensor &A, const Tensor &zi, const Tensor &x) {
  TORCH_CHECK(x.dim() == 2, "x must be a 2D tensor (batch, time)");
  TORCH_CHECK(zi.dim() == 1 && zi.size(0) == x.size(0), "zi must be a vector with x's batch size");
  TORCH_CHECK(A.dim() == 1 || A.dim() == 2, "A must be a 1D (shared) or 2D tensor");
  TORCH_CHECK(A.size(-1) == x.size(1), "A's last dimension must match x's time dimension");
  if (A.dim() == 2) TORCH_CHECK(A.size(0) == x.size(0), "If A is 2D, its first dimension must match x's batch size.");
}

Tensor recur_hip(const Tensor &A, const Tensor &zi, const Tensor &x) {
  check_common("recur", A, zi, x);
  check_recur(A, zi, x);
  if (is_half(x.scalar_type()))
    return recur_hip(A.to(at::kFloat), zi.to(at::kFloat), x.to(at::kFloat)).to(x.scalar_type());
  return run_fwd("recur", phs_recur_fwd, PHS_OP_RECUR, A, A.dim() == 1, zi, x);
}

Triple recur_backward_hip(const Tensor &A, const Tensor &zi, const Tensor &y, const Tensor &gy) {
  check_common("recur_backward", A, zi, y);
  check_recur(A, zi, y);
  TORCH_CHECK(gy.sizes() == y.sizes(), "grad_y must have y's shape");
  if (is_half(y.scalar_type()))
    return to_dtype(recur_backward_hip(A.to(at::kFloat), zi.to(at::kFloat), y.to(at::kFloat),
                                       gy.to(at::kFloat)),
                    y.scalar_type());
  return run_bwd("recur_backward", phs_recur_bwd, PHS_OP_RECUR, A, A.dim() == 1, zi, y,
                 gy.to(y.scalar_type()));
}

// ------------------------------------------------------------ LPV MxM (M = 1, 2)
void check_recurN(const Tensor &A, const Tensor &zi, const Tensor &x) {
  // host_recurN.cpp:244-248 and the fake kernel philtorch/__init__.py:179-198
  TORCH_CHECK(A.dim() == 3 || A.dim() == 4, "A must be a 3D or 4D tensor");
  TORCH_CHECK(x.dim() == 3, "x must be a 3D tensor (batch, time, order)");
  TORCH_CHECK(x.size(2) == A.size(-1), "Last dimension of x must match last dimension of A");
  TORCH_CHECK(A.size(-1) == A.size(-2), "Last two dimensions of A must be equal");
  TORCH_CHECK(zi.dim() == 2 && zi.size(1) == x.size(2) && zi.size(0) == x.size(0),
              "zi must be (batch, order)");
  TORCH_CHECK(x.size(1) == A.size(-3), "x's second dimension must match A's last-3 dimension.");
  if (A.dim() == 4)
    TORCH_CHECK(A.size(0) == x.size(0), "If A is 4D, its first dimension must match x's batch size.");
}

// [B,T,1,1] -> [B,T]; shared [T,1,1] -> [T]
std::vector<int64_t> scalar_coef_shape(const Tensor &A, bool shared) {
  return shared ? std::vector<int64_t>{A.size(0)} : std::vector<int64_t>{A.size(0), A.size(1)};
}

Tensor recurN_hip(const Tensor &A, const Tensor &zi, const Tensor &x) {
  check_common("recurN", A, zi, x);
  check_recurN(A, zi, x);
  if (is_half(x.scalar_type()))
    return recurN_hip(A.to(at::kFloat), zi.to(at::kFloat), x.to(at::kFloat)).to(x.scalar_type());
  const int64_t M = A.size(-1);
  const bool shared = A.dim() == 3;
  if (M == 1)
    return run_fwd("recurN", phs_recur_fwd, PHS_OP_RECUR, A.reshape(scalar_coef_shape(A, shared)),
                   shared, zi.reshape({zi.size(0)}), x.reshape({x.size(0), x.size(1)}))
        .view(x.sizes());
  if (M == 2) return run_fwd("recurN", phs_recur2_fwd, PHS_OP_RECUR2, A, shared, zi, x);
  TORCH_CHECK(M <= kMaxOrder, "philtorch::recurN on HIP devices supports M x M matrices up to M = ", kMaxOrder,
              ", got ", M, "x", M);
  return run_fwd_n("recurN", phs_recurN_fwd, PHS_OP_RECURN, int(M), A, shared, zi, x);
}

Tensor recur2_hip(const Tensor &A, const Tensor &zi, const Tensor &x) {
  TORCH_CHECK(A.dim() >= 2 && A.size(-1) == 2 && A.size(-2) == 2, "A must be square.");
  return recurN_hip(A, zi, x);
}

Triple recurN_backward_hip(const Tensor &A, const Tensor &zi, const Tensor &y, const Tensor &gy) {
  check_common("recurN_backward", A, zi, y);
  check_recurN(A, zi, y);
  TORCH_CHECK(gy.sizes() == y.sizes(), "grad_y must have y's shape");
  if (is_half(y.scalar_type()))
    return to_dtype(recurN_backward_hip(A.to(at::kFloat), zi.to(at::kFloat), y.to(at::kFloat),
                                        gy.to(at::kFloat)),
                    y.scalar_type());
  const int64_t M = A.size(-1);
  const bool shared = A.dim() == 3;
  const Tensor g = gy.to(y.scalar_type());
  if (M == 1) {
    auto r = run_bwd("recurN_backward", phs_recur_bwd, PHS_OP_RECUR,
                     A.reshape(scalar_coef_shape(A, shared)),
                     shared, zi.reshape({zi.size(0)}), y.reshape({y.size(0), y.size(1)}),
                     g.reshape({y.size(0), y.size(1)}));
    return {std::get<0>(r).view(A.sizes()), std::get<1>(r).view(zi.sizes()),
            std::get<2>(r).view(y.sizes())};
  }
  if (M == 2) return run_bwd("recurN_backward", phs_recur2_bwd, PHS_OP_RECUR2, A, shared, zi, y, g);
  TORCH_CHECK(M <= kMaxOrder, "philtorch::recurN on HIP devices supports M x M matrices up to M = ", kMaxOrder,
              ", got ", M, "x", M);
  return run_bwd_n("recurN_backward", phs_recurN_bwd, PHS_OP_RECURN, int(M), A, shared, zi, y, g);
}

// ------------------------------------------------------------ LTI scalar
void check_lti_recur(const Tensor &A, const Tensor &zi, const Tensor &x) {
  // host_lti_recur.cpp:49-50 and philtorch/__init__.py:233-244
  TORCH_CHECK(A.dim() <= 1, "A must be a vector or a scalar");
  TORCH_CHECK(zi.dim() == 1, "zi must be a vector");
  TORCH_CHECK(x.dim() == 2, "x must be a 2D tensor (batch, time)");
  TORCH_CHECK(zi.size(0) == x.size(0), "x and zi must have the same batch size.");
  const bool batched = A.dim() == 1 && A.numel() == x.size(0);
  TORCH_CHECK(batched || A.numel() == 1, "If A is 1D, its length must match x's batch size.");
}

bool lti_shared(const Tensor &A, const Tensor &x) { return !(A.dim() == 1 && A.numel() == x.size(0)); }

Tensor lti_recur_hip(const Tensor &A, const Tensor &zi, const Tensor &x) {
  check_common("lti_recur", A, zi, x);
  check_lti_recur(A, zi, x);
  if (is_half(x.scalar_type()))
    return lti_recur_hip(A.to(at::kFloat), zi.to(at::kFloat), x.to(at::kFloat)).to(x.scalar_type());
  return run_fwd("lti_recur", phs_lti_recur_fwd, PHS_OP_LTI_RECUR, A, lti_shared(A, x), zi, x);
}

Triple lti_recur_backward_hip(const Tensor &A, const Tensor &zi, const Tensor &y, const Tensor &gy) {
  check_common("lti_recur_backward", A, zi, y);
  check_lti_recur(A, zi, y);
  TORCH_CHECK(gy.sizes() == y.sizes(), "grad_y must have y's shape");
  if (is_half(y.scalar_type()))
    return to_dtype(lti_recur_backward_hip(A.to(at::kFloat), zi.to(at::kFloat), y.to(at::kFloat),
                                           gy.to(at::kFloat)),
                    y.scalar_type());
  return run_bwd("lti_recur_backward", phs_lti_recur_bwd, PHS_OP_LTI_RECUR, A, lti_shared(A, y), zi,
                 y, gy.to(y.scalar_type()));
}

// ------------------------------------------------------------ LTI MxM (M = 1, 2)
void check_lti_recurN(const Tensor &A, const Tensor &zi, const Tensor &x) {
  // host_lti_recurN.cpp:67-75 and philtorch/__init__.py:200-231
  TORCH_CHECK(A.dim() == 2 || A.dim() == 3, "A must be a 2D or 3D tensor");
  TORCH_CHECK(x.dim() == 3, "x must be a 3D tensor (batch, time, order)");
  TORCH_CHECK(x.size(2) == A.size(-1), "Last dimension of x must match last dimension of A");
  TORCH_CHECK(A.size(-1) == A.size(-2), "Last two dimensions of A must be equal");
  TORCH_CHECK(zi.dim() == 2 && zi.size(1) == x.size(2) && zi.size(0) == x.size(0),
              "zi must be (batch, order)");
  if (A.dim() == 3)
    TORCH_CHECK(A.size(0) == x.size(0), "If A is 3D, its first dimension must match x's batch size.");
}

Tensor lti_recurN_hip(const Tensor &A, const Tensor &zi, const Tensor &x) {
  check_common("lti_recurN", A, zi, x);
  check_lti_recurN(A, zi, x);
  if (is_half(x.scalar_type()))
    return lti_recurN_hip(A.to(at::kFloat), zi.to(at::kFloat), x.to(at::kFloat)).to(x.scalar_type());
  const int64_t M = A.size(-1);
  const bool shared = A.dim() == 2;
  if (M == 1)
    return run_fwd("lti_recurN", phs_lti_recur_fwd, PHS_OP_LTI_RECUR,
                   shared ? A.reshape({1}) : A.reshape({A.size(0)}), shared,
                   zi.reshape({zi.size(0)}), x.reshape({x.size(0), x.size(1)}))
        .view(x.sizes());
  if (M == 2) return run_fwd("lti_recurN", phs_lti_recur2_fwd, PHS_OP_LTI_RECUR2, A, shared, zi, x);
  TORCH_CHECK(M <= kMaxOrder, "philtorch::lti_recurN on HIP devices supports M x M matrices up to M = ", kMaxOrder,
              ", got ", M, "x", M);
  return run_fwd_n("lti_recurN", phs_lti_recurN_fwd, PHS_OP_LTI_RECURN, int(M), A, shared, zi, x);
}

Tensor lti_recur2_hip(const Tensor &A, const Tensor &zi, const Tensor &x) {
  TORCH_CHECK(A.dim() >= 2 && A.size(-1) == 2 && A.size(-2) == 2, "A must be square.");
  return lti_recurN_hip(A, zi, x);
}

Triple lti_recurN_backward_hip(const Tensor &A, const Tensor &zi, const Tensor &y,
                               const Tensor &gy) {
  check_common("lti_recurN_backward", A, zi, y);
  check_lti_recurN(A, zi, y);
  TORCH_CHECK(gy.sizes() == y.sizes(), "grad_y must have y's shape");
  if (is_half(y.scalar_type()))
    return to_dtype(lti_recurN_backward_hip(A.to(at::kFloat), zi.to(at::kFloat),
                                            y.to(at::kFloat), gy.to(at::kFloat)),
                    y.scalar_type());
  const int64_t M = A.size(-1);
  const bool shared = A.dim() == 2;
  const Tensor g = gy.to(y.scalar_type());
  if (M == 1) {
    auto r = run_bwd("lti_recurN_backward", phs_lti_recur_bwd, PHS_OP_LTI_RECUR,
                     shared ? A.reshape({1}) : A.reshape({A.size(0)}), shared,
                     zi.reshape({zi.size(0)}), y.reshape({y.size(0), y.size(1)}),
                     g.reshape({y.size(0), y.size(1)}));
    return {std::get<0>(r).view(A.sizes()), std::get<1>(r).view(zi.sizes()),
            std::get<2>(r).view(y.sizes())};
  }
  if (M == 2) return run_bwd("lti_recurN_backward", phs_lti_recur2_bwd, PHS_OP_LTI_RECUR2, A, shared, zi, y, g);
  TORCH_CHECK(M <= kMaxOrder, "philtorch::lti_recurN on HIP devices supports M x M matrices up to M = ", kMaxOrder,
              ", got ", M, "x", M);
  return run_bwd_n("lti_recurN_backward", phs_lti_recurN_bwd, PHS_OP_LTI_RECURN, int(M), A, shared, zi, y, g);
}

// ------------------------------------------------------------ SOS cascade
// sosfilt: fused cascade of second-order sections (scipy.signal.sosfilt
// semantics, phs_sosfilt_* in philscan.h); no counterpart op in the reference.
constexpr int64_t kSosMaxSections = 8;

void check_sos(const char *op, const Tensor &sos, const Tensor &x) {
  TORCH_CHECK(x.dim() == 2, "philtorch::", op, ": x must be a 2D tensor (batch, time)");
  TORCH_CHECK((sos.dim() == 2 || sos.dim() == 3) && sos.size(-1) == 6, "philtorch::", op,
              ": sos must be (sections, 6) or (batch, sections, 6)");
  if (sos.dim() == 3)
    TORCH_CHECK(sos.size(0) == x.size(0), "philtorch::", op, ": a 3D sos must have x's batch size");
  const int64_t S = sos.size(-2);
  TORCH_CHECK(S >= 1 && S <= kSosMaxSections, "philtorch::", op, ": 1 to ", kSosMaxSections,
              " sections per call, got ", S);
  TORCH_CHECK(sos.scalar_type() == x.scalar_type(), "sos must have the same scalar type as input");
  TORCH_CHECK(x.scalar_type() == at::kFloat || x.scalar_type() == at::kDouble, "philtorch::", op,
              ": float32 or float64 only, got ", x.scalar_type());
  TORCH_CHECK(x.is_cuda() && sos.is_cuda(), "philtorch::", op, ": philtorch_amd runs on HIP devices only (got ",
              x.device(), ")");
  TORCH_CHECK(sos.device() == x.device(), "philtorch::", op, ": all tensors must be on the same device");
}

void check_states(const char *op, const char *what, const Tensor &z, const Tensor &x, int64_t S) {
  TORCH_CHECK(z.dim() == 3 && z.size(0) == x.size(0) && z.size(1) == S && z.size(2) == 2, "philtorch::", op,
              ": ", what, " must be (batch, sections, 2)");
  TORCH_CHECK(z.scalar_type() == x.scalar_type(), "philtorch::", op, ": ", what, " must have x's scalar type");
  TORCH_CHECK(z.device() == x.device(), "philtorch::", op, ": all tensors must be on the same device");
}

// forward checkpoints per row and section (one fp64 pair each; the
// interval is the library's, per dtype)
int64_t sos_n_ckpt(int dt, int64_t T) { return int64_t(phs_sosfilt_ckpt_size(dt, 1, T, 1) / (2 * sizeof(double))); }

Triple sosfilt_hip(const Tensor &sos, const std::optional<Tensor> &zi, const Tensor &x) {
  check_sos("sosfilt", sos, x);
  const int64_t B = x.size(0), T = x.size(1), S = sos.size(-2);
  if (zi) check_states("sosfilt", "zi", *zi, x, S);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  const int dt = phs_dtype_of(x.scalar_type());
  Tensor sc = sos.contiguous(), xc = x.contiguous();
  Tensor zc = zi ? zi->contiguous() : Tensor();
  Tensor y = at::empty_like(xc, at::MemoryFormat::Contiguous);
  Tensor zf = at::empty({B, S, 2}, x.options());
  Tensor ckpt = at::empty({B, S, sos_n_ckpt(dt, T), 2}, x.options().dtype(at::kDouble));
  TORCH_CHECK(size_t(ckpt.numel()) * sizeof(double) == phs_sosfilt_ckpt_size(dt, B, T, int(S)),
              "philtorch::sosfilt: checkpoint layout mismatch with libphilscan");
  if (B == 0 || T == 0) {
    if (zi) zf.copy_(zc); else zf.zero_();
    return {y, zf, ckpt};
  }
  void *stream = stream_of(x);
  const Workspace ws = workspace_for(x, phs_sosfilt_workspace_size(dt, B, T, int(S), 0), stream);
  check_status(phs_sosfilt_fwd(dt, B, T, int(S), sc.const_data_ptr(), sos.dim() == 2 ? 1 : 0,
                               zi ? zc.const_data_ptr() : nullptr, xc.const_data_ptr(), y.mutable_data_ptr(),
                               zf.mutable_data_ptr(), ckpt.mutable_data_ptr(), ws.ptr, ws.bytes, stream),
               "sosfilt");
  return {y, zf, ckpt};
}

// Returns (grad_x, grad_sos, grad_zi); grad_sos is zero unless need_sos.
Triple sosfilt_backward_hip(const Tensor &sos, const Tensor &x, const Tensor &ckpt, const Tensor &gy,
                            const std::optional<Tensor> &gzf, bool need_sos) {
  check_sos("sosfilt_backward", sos, x);
  const int64_t B = x.size(0), T = x.size(1), S = sos.size(-2);
  TORCH_CHECK(gy.sizes() == x.sizes(), "philtorch::sosfilt_backward: grad_y must have x's shape");
  TORCH_CHECK(gy.device() == x.device(), "philtorch::sosfilt_backward: all tensors must be on the same device");
  if (gzf) check_states("sosfilt_backward", "grad_zf", *gzf, x, S);
  const int64_t nck = sos_n_ckpt(phs_dtype_of(x.scalar_type()), T);
  TORCH_CHECK(ckpt.scalar_type() == at::kDouble && ckpt.dim() == 4 && ckpt.size(0) == B && ckpt.size(1) == S &&
                  ckpt.size(2) == nck && ckpt.size(3) == 2 && ckpt.device() == x.device(),
              "philtorch::sosfilt_backward: ckpt must be the forward's checkpoint tensor");
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  const int dt = phs_dtype_of(x.scalar_type());
  Tensor sc = sos.contiguous(), xc = x.contiguous(), gc = gy.to(x.scalar_type()).contiguous();
  Tensor cc = ckpt.contiguous();
  Tensor gzc = gzf ? gzf->contiguous() : Tensor();
  Tensor gx = at::empty_like(xc, at::MemoryFormat::Contiguous);
  Tensor gsos = need_sos ? at::empty(sos.sizes(), sos.options()) : at::zeros(sos.sizes(), sos.options());
  Tensor gzi = at::empty({B, S, 2}, x.options());
  if (B == 0 || T == 0) {
    if (need_sos) gsos.zero_();
    if (gzf) gzi.copy_(gzc); else gzi.zero_();
    return {gx, gsos, gzi};
  }
  void *stream = stream_of(x);
  const Workspace ws = workspace_for(x, phs_sosfilt_workspace_size(dt, B, T, int(S), 1), stream);
  check_status(phs_sosfilt_bwd(dt, B, T, int(S), sc.const_data_ptr(), sos.dim() == 2 ? 1 : 0,
                               need_sos ? xc.const_data_ptr() : nullptr, need_sos ? cc.const_data_ptr() : nullptr,
                               gc.const_data_ptr(), gzf ? gzc.const_data_ptr() : nullptr, gx.mutable_data_ptr(),
                               need_sos ? gsos.mutable_data_ptr() : nullptr, gzi.mutable_data_ptr(), ws.ptr,
                               ws.bytes, stream),
               "sosfilt_backward");
  return {gx, gsos, gzi};
}

// One biquad as lfilter(b, a, x, zi, form="tdf2") on the cascade kernel
// with b and a read where they lie (phs_biquad_fwd): b (nb,) or (batch, nb),
// nb <= 3; a (2,) or (batch, 2), the denominator after its leading 1, each
// with unit inner stride (any row stride: a column slice of a coefficient
// table needs no copy); zi None or (batch, 2).  Returns (y, zf, ckpt), ckpt
// the forward's state checkpoints for the backward.
void check_biquad(const char *op, const Tensor &b, const Tensor &a, const Tensor &x) {
  TORCH_CHECK(x.dim() == 2, "philtorch::", op, ": x must be a 2D tensor (batch, time)");
  TORCH_CHECK(b.dim() == a.dim() && (b.dim() == 1 || b.dim() == 2), "philtorch::", op,
              ": b and a must both be 1D (shared) or both 2D (batch, taps)");
  TORCH_CHECK(b.size(-1) >= 1 && b.size(-1) <= 3 && a.size(-1) == 2, "philtorch::", op,
              ": a biquad: b of 1 to 3 taps, a of 2 after the leading 1");
  if (b.dim() == 2)
    TORCH_CHECK(b.size(0) == x.size(0) && a.size(0) == x.size(0), "philtorch::", op,
                ": 2D b and a must have x's batch size");
  TORCH_CHECK(b.scalar_type() == x.scalar_type() && a.scalar_type() == x.scalar_type(), "philtorch::", op,
              ": b, a and x must have the same scalar type");
  TORCH_CHECK(x.scalar_type() == at::kFloat || x.scalar_type() == at::kDouble, "philtorch::", op,
              ": float32 or float64 only, got ", x.scalar_type());
  TORCH_CHECK(x.is_cuda() && b.device() == x.device() && a.device() == x.device(), "philtorch::", op,
              ": philtorch_amd runs on HIP devices only, all tensors on one device");
}

// b or a with unit inner stride (a copy only where the taps are strided);
// its row stride in elements, 0 for a shared (1D) one
Tensor rows_unit_inner(const Tensor &t, int64_t &row_stride) {
  Tensor u = t;
  if (u.stride(-1) != 1 || (u.dim() == 2 && u.size(0) > 1 && u.stride(0) == 0)) u = u.contiguous();
  row_stride = (u.dim() == 2 && u.size(0) > 1) ? u.stride(0) : 0;
  return u;
}

Triple biquad_hip(const Tensor &b, const Tensor &a, const std::optional<Tensor> &zi, const Tensor &x) {
  check_biquad("biquad", b, a, x);
  const int64_t B = x.size(0), T = x.size(1);
  if (zi)
    TORCH_CHECK(zi->dim() == 2 && zi->size(0) == B && zi->size(1) == 2 && zi->scalar_type() == x.scalar_type() &&
                    zi->device() == x.device(),
                "philtorch::biquad: zi must be (batch, 2) with x's scalar type");
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  const int dt = phs_dtype_of(x.scalar_type());
  int64_t bs = 0, as = 0;
  Tensor bu = rows_unit_inner(b, bs), au = rows_unit_inner(a, as), xc = x.contiguous();
  Tensor zc = zi ? zi->contiguous() : Tensor();
  Tensor y = at::empty_like(xc, at::MemoryFormat::Contiguous);
  Tensor zf = at::empty({B, 2}, x.options());
  Tensor ckpt = at::empty({B, 1, sos_n_ckpt(dt, T), 2}, x.options().dtype(at::kDouble));
  if (B == 0 || T == 0) {
    if (zi) zf.copy_(zc); else zf.zero_();
    return {y, zf, ckpt};
  }
  void *stream = stream_of(x);
  const Workspace ws = workspace_for(x, phs_sosfilt_workspace_size(dt, B, T, 1, 0), stream);
  check_status(phs_biquad_fwd(dt, B, T, bu.const_data_ptr(), int(b.size(-1)), bs, au.const_data_ptr(), as,
                              zi ? zc.const_data_ptr() : nullptr, xc.const_data_ptr(), y.mutable_data_ptr(),
                              zf.mutable_data_ptr(), ckpt.mutable_data_ptr(), ws.ptr, ws.bytes, stream),
               "biquad");
  return {y, zf, ckpt};
}

// Column `col` of a coefficient table along its second-to-last dimension
// (b [B, C, nb] or [C, nb]: the C4 caller's b[:, s]); col -1: t itself.
Tensor table_column(const Tensor &t, int64_t col, const char *op) {
  if (col < 0) return t;
  TORCH_CHECK(t.dim() >= 2 && col < t.size(-2), "philtorch::", op, ": column ", col, " of a table of ",
              t.dim() >= 2 ? t.size(-2) : 0, " columns");
  return t.select(-2, col);
}

// Gradients of biquad (phs_biquad_bwd_cols): (grad_x, grad_bt, grad_at,
// grad_zi) for b = bt's column b_col (bt itself for -1) and a likewise;
// grad_bt, grad_at shaped like bt and at, the biquad's gradient in its
// column and zeros elsewhere (all zero unless need_coef); grad_zf None is
// zero.
std::vector<Tensor> biquad_backward_impl(const char *op, const Tensor &bt, int64_t b_col, const Tensor &at_,
                                         int64_t a_col, const Tensor &x, const Tensor &ckpt, const Tensor &gy,
                                         const std::optional<Tensor> &gzf, bool need_coef) {
  const Tensor b = table_column(bt, b_col, op), a = table_column(at_, a_col, op);
  check_biquad(op, b, a, x);
  const int64_t B = x.size(0), T = x.size(1);
  TORCH_CHECK(gy.sizes() == x.sizes() && gy.device() == x.device(),
              "philtorch::biquad_backward: grad_y must have x's shape and device");
  if (gzf)
    TORCH_CHECK(gzf->dim() == 2 && gzf->size(0) == B && gzf->size(1) == 2 && gzf->device() == x.device(),
                "philtorch::biquad_backward: grad_zf must be (batch, 2)");
  const int64_t nck = sos_n_ckpt(phs_dtype_of(x.scalar_type()), T);
  TORCH_CHECK(ckpt.scalar_type() == at::kDouble && ckpt.dim() == 4 && ckpt.size(0) == B && ckpt.size(1) == 1 &&
                  ckpt.size(2) == nck && ckpt.size(3) == 2 && ckpt.device() == x.device(),
              "philtorch::biquad_backward: ckpt must be the forward's checkpoint tensor");
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  const int dt = phs_dtype_of(x.scalar_type());
  int64_t bs = 0, as = 0;
  Tensor bu = rows_unit_inner(b, bs), au = rows_unit_inner(a, as), xc = x.contiguous();
  Tensor gc = gy.to(x.scalar_type()).contiguous(), cc = ckpt.contiguous();
  Tensor gzc = gzf ? gzf->to(x.scalar_type()).contiguous() : Tensor();
  Tensor gx = at::empty_like(xc, at::MemoryFormat::Contiguous);
  Tensor gb = need_coef ? at::empty(bt.sizes(), bt.options()) : at::zeros(bt.sizes(), bt.options());
  Tensor ga = need_coef ? at::empty(at_.sizes(), at_.options()) : at::zeros(at_.sizes(), at_.options());
  Tensor gzi = at::empty({B, 2}, x.options());
  if (B == 0 || T == 0) {
    if (need_coef) gb.zero_(), ga.zero_();
    if (gzf) gzi.copy_(gzc); else gzi.zero_();
    return {gx, gb, ga, gzi};
  }
  void *stream = stream_of(x);
  const Workspace ws = workspace_for(x, phs_sosfilt_workspace_size(dt, B, T, 1, 1), stream);
  const int b_cols = b_col >= 0 ? int(bt.size(-2)) : 1, a_cols = a_col >= 0 ? int(at_.size(-2)) : 1;
  check_status(phs_biquad_bwd_cols(dt, B, T, bu.const_data_ptr(), int(b.size(-1)), bs, au.const_data_ptr(), as,
                                   need_coef ? xc.const_data_ptr() : nullptr,
                                   need_coef ? cc.const_data_ptr() : nullptr, gc.const_data_ptr(),
                                   gzf ? gzc.const_data_ptr() : nullptr, gx.mutable_data_ptr(),
                                   need_coef ? gb.mutable_data_ptr() : nullptr, b_cols, int(b_col < 0 ? 0 : b_col),
                                   need_coef ? ga.mutable_data_ptr() : nullptr, a_cols, int(a_col < 0 ? 0 : a_col),
                                   gzi.mutable_data_ptr(), ws.ptr, ws.bytes, stream),
               op);
  return {gx, gb, ga, gzi};
}

std::vector<Tensor> biquad_backward_hip(const Tensor &b, const Tensor &a, const Tensor &x, const Tensor &ckpt,
                                        const Tensor &gy, const std::optional<Tensor> &gzf, bool need_coef) {
  return biquad_backward_impl("biquad_backward", b, -1, a, -1, x, ckpt, gy, gzf, need_coef);
}

// biquad with b and a given as columns of coefficient tables (col -1: the
// coefficients themselves), so that autograd's gradient of a table needs no
// zero-filled copy and column write per call: (y, zf, ckpt)
Triple biquad_cols_hip(const Tensor &bt, int64_t b_col, const Tensor &at_, int64_t a_col,
                       const std::optional<Tensor> &zi, const Tensor &x) {
  return biquad_hip(table_column(bt, b_col, "biquad_cols"), table_column(at_, a_col, "biquad_cols"), zi, x);
}

std::vector<Tensor> biquad_cols_backward_hip(const Tensor &bt, int64_t b_col, const Tensor &at_, int64_t a_col,
                                             const Tensor &x, const Tensor &ckpt, const Tensor &gy,
                                             const std::optional<Tensor> &gzf, bool need_coef) {
  return biquad_backward_impl("biquad_cols_backward", bt, b_col, at_, a_col, x, ckpt, gy, gzf, need_coef);
}

// Zero-phase filter of order 4 at most (phs_filtfilt_fwd;
// philtorch/lti/filtering.py:413-484): b (nb,) or (batch, nb), nb <= 5; a
// (na,) or (batch, na), the denominator after its leading 1, na <= 4;
// padmode a phs_padmode code.  Its gradients are filtfilt_backward below.
void filtfilt_check(const char *op, const Tensor &b, const Tensor &a, const Tensor &x, int64_t padmode,
                    int64_t padlen) {
  TORCH_CHECK(x.dim() == 2, op, ": x must be a 2D tensor (batch, time)");
  TORCH_CHECK(b.dim() == a.dim() && (b.dim() == 1 || b.dim() == 2), op, ": b and a must both be 1D "
              "(shared) or both 2D (batch, taps)");
  const int64_t B = x.size(0), T = x.size(1);
  if (b.dim() == 2) TORCH_CHECK(b.size(0) == B && a.size(0) == B, op, ": 2D b and a must have x's batch size");
  const int64_t nb = b.size(-1), na = a.size(-1);
  TORCH_CHECK(nb >= 1 && nb <= 5 && na >= 1 && na <= 4, op, ": filters of order 4 at most "
              "(b: 1 to 5 taps, a: 1 to 4 after the leading 1)");
  TORCH_CHECK(b.scalar_type() == x.scalar_type() && a.scalar_type() == x.scalar_type(), op,
              ": b, a and x must have the same scalar type");
  TORCH_CHECK(x.scalar_type() == at::kFloat || x.scalar_type() == at::kDouble, op,
              ": float32 or float64 only, got ", x.scalar_type());
  TORCH_CHECK(x.is_cuda() && b.device() == x.device() && a.device() == x.device(), op,
              ": philtorch_amd runs on HIP devices only, all tensors on one device");
  TORCH_CHECK(padmode >= PHS_PAD_CONSTANT && padmode <= PHS_PAD_CIRCULAR, op, ": unknown padmode ", padmode);
  TORCH_CHECK(padlen >= 0 && T > padlen, "Input signal length ", T, " must be greater than pad length ", padlen, ".");
}

// filtfilt that also returns what its coefficient backward would compute
// again (phs_filtfilt_fwd_hs): (y, mid, h1, h2) with mid pass 1's output and
// final state (bytes, phs_filtfilt_mid_size) and h1, h2 (batch, T, order)
// both passes' states.
std::tuple<Tensor, Tensor, Tensor, Tensor> filtfilt_states_hip(const Tensor &b, const Tensor &a, const Tensor &x,
                                                               int64_t padmode, int64_t padlen) {
  filtfilt_check("philtorch::filtfilt_states", b, a, x, padmode, padlen);
  const int64_t B = x.size(0), T = x.size(1), nb = b.size(-1), na = a.size(-1);
  const int64_t M = std::max(nb - 1, na);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  const int dt = phs_dtype_of(x.scalar_type());
  Tensor bc = b.contiguous(), ac = a.contiguous(), xc = x.contiguous();
  Tensor y = at::empty_like(xc, at::MemoryFormat::Contiguous);
  Tensor mid = at::empty({int64_t(B == 0 ? 0 : phs_filtfilt_mid_size(dt, B, T))}, x.options().dtype(at::kByte));
  Tensor h1 = at::empty({B, T, M}, x.options()), h2 = at::empty({B, T, M}, x.options());
  if (B == 0) return {y, mid, h1, h2};
  void *stream = stream_of(x);
  const Workspace ws = workspace_for(x, phs_filtfilt_workspace_size(dt, B, T), stream);
  check_status(phs_filtfilt_fwd_hs(dt, B, T, bc.const_data_ptr(), int(nb), ac.const_data_ptr(), int(na),
                                   b.dim() == 1 ? 1 : 0, int(padmode), padlen, xc.const_data_ptr(),
                                   y.mutable_data_ptr(), mid.mutable_data_ptr(), h1.mutable_data_ptr(),
                                   h2.mutable_data_ptr(), ws.ptr, ws.bytes, stream),
               "filtfilt_states");
  return {y, mid, h1, h2};
}

Tensor filtfilt_hip(const Tensor &b, const Tensor &a, const Tensor &x, int64_t padmode, int64_t padlen) {
  filtfilt_check("philtorch::filtfilt", b, a, x, padmode, padlen);
  const int64_t B = x.size(0), T = x.size(1), nb = b.size(-1), na = a.size(-1);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  const int dt = phs_dtype_of(x.scalar_type());
  Tensor bc = b.contiguous(), ac = a.contiguous(), xc = x.contiguous();
  Tensor y = at::empty_like(xc, at::MemoryFormat::Contiguous);
  if (B == 0) return y;
  Tensor mid = at::empty({int64_t(phs_filtfilt_mid_size(dt, B, T))}, x.options().dtype(at::kByte));
  void *stream = stream_of(x);
  const Workspace ws = workspace_for(x, phs_filtfilt_workspace_size(dt, B, T), stream);
  check_status(phs_filtfilt_fwd(dt, B, T, bc.const_data_ptr(), int(nb), ac.const_data_ptr(), int(na),
                                b.dim() == 1 ? 1 : 0, int(padmode), padlen, xc.const_data_ptr(), y.mutable_data_ptr(),
                                mid.mutable_data_ptr(), ws.ptr, ws.bytes, stream),
               "filtfilt");
  return y;
}

// Gradients of filtfilt (phs_filtfilt_bwd): [grad_x, grad_b, grad_a] for
// grad_y (batch, time), b, a and x as filtfilt's; grad_b and grad_a are
// empty unless need_coef (x is read only then: the map is linear in x).
std::vector<Tensor> filtfilt_backward_hip(const Tensor &b, const Tensor &a, const Tensor &x, const Tensor &grad_y,
                                          int64_t padmode, int64_t padlen, bool need_coef,
                                          const std::optional<Tensor> &mid, const std::optional<Tensor> &h1,
                                          const std::optional<Tensor> &h2) {
  TORCH_CHECK(bool(mid) == bool(h1) && bool(h1) == bool(h2),
              "philtorch::filtfilt_backward: mid, h1 and h2 come together (filtfilt_states) or not at all");
  filtfilt_check("philtorch::filtfilt_backward", b, a, grad_y, padmode, padlen);
  TORCH_CHECK(x.sizes() == grad_y.sizes() && x.scalar_type() == grad_y.scalar_type() &&
                  x.device() == grad_y.device(),
              "philtorch::filtfilt_backward: x and grad_y must have the same shape, type and device");
  const int64_t B = grad_y.size(0), T = grad_y.size(1), nb = b.size(-1), na = a.size(-1);
  const int M = int(std::max(nb - 1, na));
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(grad_y.device());
  const int dt = phs_dtype_of(grad_y.scalar_type());
  Tensor bc = b.contiguous(), ac = a.contiguous(), gy = grad_y.contiguous();
  Tensor xc = need_coef ? x.contiguous() : x;
  Tensor gx = at::empty_like(gy, at::MemoryFormat::Contiguous);
  Tensor gb = need_coef ? at::empty_like(bc) : at::empty({0}, b.options());
  Tensor ga = need_coef ? at::empty_like(ac) : at::empty({0}, a.options());
  if (B == 0) return {gx, gb, ga};
  Tensor scratch = at::empty({int64_t(phs_filtfilt_bwd_scratch_size(dt, M, B, T, padlen, need_coef ? 1 : 0))},
                             gy.options().dtype(at::kByte));
  void *stream = stream_of(gy);
  const Workspace ws = workspace_for(gy, phs_filtfilt_workspace_size(dt, B, T), stream);
  const bool kept = need_coef && mid && h1 && h2;
  if (kept)
    TORCH_CHECK(mid->numel() == int64_t(phs_filtfilt_mid_size(dt, B, T)) && h1->dim() == 3 && h1->size(0) == B &&
                    h1->size(1) == T && h1->size(2) == M && h2->sizes() == h1->sizes() &&
                    h1->scalar_type() == grad_y.scalar_type() && h2->scalar_type() == grad_y.scalar_type() &&
                    mid->is_contiguous() && h1->is_contiguous() && h2->is_contiguous(),
                "philtorch::filtfilt_backward: mid, h1, h2 must be filtfilt_states' outputs for these shapes");
  check_status(phs_filtfilt_bwd_hs(dt, B, T, bc.const_data_ptr(), int(nb), ac.const_data_ptr(), int(na),
                                b.dim() == 1 ? 1 : 0, int(padmode), padlen, need_coef ? xc.const_data_ptr() : nullptr,
                                kept ? mid->const_data_ptr() : nullptr, kept ? h1->const_data_ptr() : nullptr,
                                kept ? h2->const_data_ptr() : nullptr,
                                gy.const_data_ptr(), gx.mutable_data_ptr(), need_coef ? gb.mutable_data_ptr() : nullptr,
                                need_coef ? ga.mutable_data_ptr() : nullptr, scratch.mutable_data_ptr(),
                                size_t(scratch.numel()), ws.ptr, ws.bytes, stream),
               "filtfilt_backward");
  return {gx, gb, ga};
}

// Single-input single-output LTI state space of order <= 4, fused
// (phs_lti_ss_fwd; philtorch/lti/ssm.py:386-589 for a 2D x): returns (y, zf).
// A (M, M) or (batch, M, M); B, C None, (M,) or (batch, M); D None, one value
// or (batch,); zi None or (batch, M); out_idx selects the output state when
// C is None; reverse runs the model backwards in time (phs_lti_ss_rev).
// lti_ss's argument checks (shared by its backward); returns M.
int64_t lti_ss_meta_check(const Tensor &A, const std::optional<Tensor> &Bm, const std::optional<Tensor> &Cm,
                          const std::optional<Tensor> &Dm, const std::optional<Tensor> &zi, const Tensor &x,
                          int64_t out_idx) {
  TORCH_CHECK(x.dim() == 2, "philtorch::lti_ss: x must be a 2D tensor (batch, time)");
  TORCH_CHECK((A.dim() == 2 || A.dim() == 3) && A.size(-1) == A.size(-2),
              "philtorch::lti_ss: A must be (M, M) or (batch, M, M)");
  const int64_t B = x.size(0), M = A.size(-1);
  TORCH_CHECK(M >= 1 && M <= kMaxOrder, "philtorch::lti_ss: state order 1 to ", kMaxOrder, ", got ", M);
  if (A.dim() == 3) TORCH_CHECK(A.size(0) == B, "philtorch::lti_ss: a 3D A must have x's batch size");
  TORCH_CHECK(x.scalar_type() == at::kFloat || x.scalar_type() == at::kDouble,
              "philtorch::lti_ss: float32 or float64 only, got ", x.scalar_type());
  TORCH_CHECK(x.is_cuda(), "philtorch::lti_ss: philtorch_amd runs on HIP devices only (got ", x.device(), ")");
  auto same = [&](const Tensor &t, const char *what) {
    TORCH_CHECK(t.scalar_type() == x.scalar_type(), "philtorch::lti_ss: ", what, " must have x's scalar type");
    TORCH_CHECK(t.device() == x.device(), "philtorch::lti_ss: all tensors must be on the same device");
  };
  same(A, "A");
  auto vec_ok = [&](const Tensor &t) { return (t.dim() == 1 && t.size(0) == M) || (t.dim() == 2 && t.size(0) == B && t.size(1) == M); };
  if (Bm) {
    same(*Bm, "B");
    TORCH_CHECK(vec_ok(*Bm), "philtorch::lti_ss: B must be (M,) or (batch, M)");
  }
  if (Cm) {
    same(*Cm, "C");
    TORCH_CHECK(vec_ok(*Cm), "philtorch::lti_ss: C must be (M,) or (batch, M)");
  } else {
    TORCH_CHECK(out_idx >= 0 && out_idx < M, "philtorch::lti_ss: out_idx must be in [0, ", M, ") when C is None");
  }
  if (Dm) {
    same(*Dm, "D");
    TORCH_CHECK(Dm->numel() == 1 || (Dm->dim() == 1 && Dm->size(0) == B),
                "philtorch::lti_ss: D must hold one value or (batch,)");
  }
  if (zi) {
    same(*zi, "zi");
    TORCH_CHECK(zi->dim() == 2 && zi->size(0) == B && zi->size(1) == M, "philtorch::lti_ss: zi must be (batch, M)");
  }
  return M;
}

// A backward's optional states argument: the forward's (batch, T, M).
void check_states(const std::optional<Tensor> &hs, const Tensor &x, int64_t M, const char *op) {
  if (hs)
    TORCH_CHECK(hs->dim() == 3 && hs->size(0) == x.size(0) && hs->size(1) == x.size(1) && hs->size(2) == M &&
                    hs->scalar_type() == x.scalar_type() && hs->device() == x.device(),
                "philtorch::", op, ": hs must be the forward's states (batch, T, M)");
}

// keep_states: also hs (batch, T, M), the state before every step, from the
// same pass (phs_lti_ss_fwd_hs) for the coefficient backward.
std::tuple<Tensor, Tensor, Tensor> lti_ss_impl(const Tensor &A, const std::optional<Tensor> &Bm,
                                               const std::optional<Tensor> &Cm, const std::optional<Tensor> &Dm,
                                               const std::optional<Tensor> &zi, const Tensor &x, int64_t out_idx,
                                               bool reverse, bool keep_states) {
  const int64_t M = lti_ss_meta_check(A, Bm, Cm, Dm, zi, x, out_idx);
  const int64_t B = x.size(0), T = x.size(1);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  const int dt = phs_dtype_of(x.scalar_type());
  Tensor Ac = A.contiguous(), xc = x.contiguous();
  Tensor bc = Bm ? Bm->contiguous() : Tensor(), cc = Cm ? Cm->contiguous() : Tensor();
  Tensor dc = Dm ? Dm->contiguous() : Tensor(), zc = zi ? zi->contiguous() : Tensor();
  Tensor y = at::empty_like(xc, at::MemoryFormat::Contiguous);
  Tensor zf = at::empty({B, M}, x.options());
  Tensor hs = at::empty({keep_states ? B : 0, keep_states ? T : 0, M}, x.options());
  if (B == 0) return {y, zf, hs};
  if (T == 0) {
    if (zi) zf.copy_(zc); else zf.zero_();
    return {y, zf, hs};
  }
  void *stream = stream_of(x);
  const Workspace ws = workspace_for(x, phs_lti_ss_workspace_size(dt, int(M), B, T), stream);
  const void *bp = Bm ? bc.const_data_ptr() : nullptr, *cp = Cm ? cc.const_data_ptr() : nullptr;
  const void *dp = Dm ? dc.const_data_ptr() : nullptr, *zp = zi ? zc.const_data_ptr() : nullptr;
  const int ash = A.dim() == 2 ? 1 : 0, bsh = Bm && Bm->dim() == 1 ? 1 : 0, csh = Cm && Cm->dim() == 1 ? 1 : 0;
  const int dsh = Dm && Dm->numel() == 1 ? 1 : 0;
  if (keep_states)
    check_status(phs_lti_ss_fwd_hs(dt, int(M), B, T, Ac.const_data_ptr(), ash, bp, bsh, cp, csh, int(out_idx), dp,
                                   dsh, zp, xc.const_data_ptr(), y.mutable_data_ptr(), zf.mutable_data_ptr(),
                                   hs.mutable_data_ptr(), reverse ? 1 : 0, ws.ptr, ws.bytes, stream),
                 "lti_ss_states");
  else
    check_status((reverse ? phs_lti_ss_rev : phs_lti_ss_fwd)(dt, int(M), B, T, Ac.const_data_ptr(), ash, bp, bsh, cp,
                                                             csh, int(out_idx), dp, dsh, zp, xc.const_data_ptr(),
                                                             y.mutable_data_ptr(), zf.mutable_data_ptr(), ws.ptr,
                                                             ws.bytes, stream),
                 "lti_ss");
  return {y, zf, hs};
}

std::tuple<Tensor, Tensor> lti_ss_hip(const Tensor &A, const std::optional<Tensor> &Bm,
                                      const std::optional<Tensor> &Cm, const std::optional<Tensor> &Dm,
                                      const std::optional<Tensor> &zi, const Tensor &x, int64_t out_idx,
                                      bool reverse) {
  auto [y, zf, hs] = lti_ss_impl(A, Bm, Cm, Dm, zi, x, out_idx, reverse, false);
  return {y, zf};
}

// lti_ss that also returns hs (batch, T, M), the states lti_ss_backward
// would compute again.
std::tuple<Tensor, Tensor, Tensor> lti_ss_states_hip(const Tensor &A, const std::optional<Tensor> &Bm,
                                                     const std::optional<Tensor> &Cm,
                                                     const std::optional<Tensor> &Dm,
                                                     const std::optional<Tensor> &zi, const Tensor &x,
                                                     int64_t out_idx, bool reverse) {
  return lti_ss_impl(A, Bm, Cm, Dm, zi, x, out_idx, reverse, true);
}

// lfilter of order <= 4 from b and a directly (phs_lfilter_fwd;
// philtorch/lti/filtering.py:211-333 in its companion-form state space):
// returns (y, zf).  b (nb,) or (batch, nb); a (na,) or (batch, na), the
// denominator after its leading 1; form 0 "tdf2", 1 "df2"; zi None or
// (batch, max(nb - 1, na)); reverse runs the filter backwards in time
// (phs_lfilter_rev).
// lfilter_ss's argument checks (shared by its backward); returns the order.
int64_t lfilter_ss_meta_check(const Tensor &b, const Tensor &a, const std::optional<Tensor> &zi, const Tensor &x,
                              int64_t form) {
  TORCH_CHECK(x.dim() == 2, "philtorch::lfilter_ss: x must be a 2D tensor (batch, time)");
  TORCH_CHECK(b.dim() == a.dim() && (b.dim() == 1 || b.dim() == 2),
              "philtorch::lfilter_ss: b and a must both be 1D (shared) or both 2D (batch, taps)");
  const int64_t B = x.size(0), nb = b.size(-1), na = a.size(-1);
  if (b.dim() == 2)
    TORCH_CHECK(b.size(0) == B && a.size(0) == B, "philtorch::lfilter_ss: 2D b and a must have x's batch size");
  const int64_t M = std::max(nb - 1, na);
  TORCH_CHECK(nb >= 1 && na >= 1 && M <= kMaxOrder, "philtorch::lfilter_ss: filters of order 1 to ", kMaxOrder);
  TORCH_CHECK(form == PHS_FORM_TDF2 || form == PHS_FORM_DF2, "philtorch::lfilter_ss: form 0 (tdf2) or 1 (df2)");
  TORCH_CHECK(b.scalar_type() == x.scalar_type() && a.scalar_type() == x.scalar_type(),
              "philtorch::lfilter_ss: b, a and x must have the same scalar type");
  TORCH_CHECK(x.scalar_type() == at::kFloat || x.scalar_type() == at::kDouble,
              "philtorch::lfilter_ss: float32 or float64 only, got ", x.scalar_type());
  TORCH_CHECK(x.is_cuda() && b.device() == x.device() && a.device() == x.device(),
              "philtorch::lfilter_ss: philtorch_amd runs on HIP devices only, all tensors on one device");
  if (zi) {
    TORCH_CHECK(zi->dim() == 2 && zi->size(0) == B && zi->size(1) == M && zi->scalar_type() == x.scalar_type() &&
                    zi->device() == x.device(),
                "philtorch::lfilter_ss: zi must be (batch, order) with x's scalar type");
  }
  return M;
}

std::tuple<Tensor, Tensor, Tensor> lfilter_ss_impl(const Tensor &b, const Tensor &a,
                                                   const std::optional<Tensor> &zi, const Tensor &x, int64_t form,
                                                   bool reverse, bool keep_states) {
  const int64_t M = lfilter_ss_meta_check(b, a, zi, x, form);
  const int64_t B = x.size(0), T = x.size(1), nb = b.size(-1), na = a.size(-1);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  const int dt = phs_dtype_of(x.scalar_type());
  Tensor bc = b.contiguous(), ac = a.contiguous(), xc = x.contiguous(), zc = zi ? zi->contiguous() : Tensor();
  Tensor y = at::empty_like(xc, at::MemoryFormat::Contiguous);
  Tensor zf = at::empty({B, M}, x.options());
  Tensor hs = at::empty({keep_states ? B : 0, keep_states ? T : 0, M}, x.options());
  if (B == 0) return {y, zf, hs};
  if (T == 0) {
    if (zi) zf.copy_(zc); else zf.zero_();
    return {y, zf, hs};
  }
  void *stream = stream_of(x);
  const Workspace ws = workspace_for(x, phs_lti_ss_workspace_size(dt, int(M), B, T), stream);
  if (keep_states)
    check_status(phs_lfilter_fwd_hs(dt, B, T, bc.const_data_ptr(), int(nb), ac.const_data_ptr(), int(na),
                                    b.dim() == 1 ? 1 : 0, int(form), zi ? zc.const_data_ptr() : nullptr,
                                    xc.const_data_ptr(), y.mutable_data_ptr(), zf.mutable_data_ptr(),
                                    hs.mutable_data_ptr(), reverse ? 1 : 0, ws.ptr, ws.bytes, stream),
                 "lfilter_ss_states");
  else
    check_status((reverse ? phs_lfilter_rev : phs_lfilter_fwd)(dt, B, T, bc.const_data_ptr(), int(nb), ac.const_data_ptr(), int(na),
                                 b.dim() == 1 ? 1 : 0, int(form), zi ? zc.const_data_ptr() : nullptr,
                                 xc.const_data_ptr(), y.mutable_data_ptr(), zf.mutable_data_ptr(), ws.ptr, ws.bytes,
                                 stream),
                 "lfilter_ss");
  return {y, zf, hs};
}

std::tuple<Tensor, Tensor> lfilter_ss_hip(const Tensor &b, const Tensor &a, const std::optional<Tensor> &zi,
                                          const Tensor &x, int64_t form, bool reverse) {
  auto [y, zf, hs] = lfilter_ss_impl(b, a, zi, x, form, reverse, false);
  return {y, zf};
}

// lfilter_ss that also returns hs (batch, T, order), the states
// lfilter_ss_backward would compute again.
std::tuple<Tensor, Tensor, Tensor> lfilter_ss_states_hip(const Tensor &b, const Tensor &a,
                                                         const std::optional<Tensor> &zi, const Tensor &x,
                                                         int64_t form, bool reverse) {
  return lfilter_ss_impl(b, a, zi, x, form, reverse, true);
}

// Gradients of lti_ss w.r.t. every input (phs_lti_ss_bwd): returns
// (grad_A, grad_B, grad_C, grad_D, grad_zi, grad_x), each shaped like its
// input (a shared operand's gradient summed over the rows; an absent
// operand's an empty tensor; grad_zi (batch, M) whether zi was given or
// not).  grad_zf None is zero.  Replaces the autograd of the composed state
// space (philtorch/lti/ssm.py:386-589).
std::vector<Tensor> lti_ss_backward_hip(const Tensor &A, const std::optional<Tensor> &Bm,
                                        const std::optional<Tensor> &Cm, const std::optional<Tensor> &Dm,
                                        const std::optional<Tensor> &zi, const Tensor &x, const Tensor &gy,
                                        const std::optional<Tensor> &gzf, int64_t out_idx, bool reverse,
                                        const std::optional<Tensor> &hs) {
  // the forward's argument checks
  (void)lti_ss_meta_check(A, Bm, Cm, Dm, zi, x, out_idx);
  const int64_t B = x.size(0), T = x.size(1), M = A.size(-1);
  check_states(hs, x, M, "lti_ss_backward");
  Tensor hc = hs ? hs->contiguous() : Tensor();
  TORCH_CHECK(gy.sizes() == x.sizes() && gy.device() == x.device(),
              "philtorch::lti_ss_backward: grad_y must have x's shape and device");
  if (gzf)
    TORCH_CHECK(gzf->dim() == 2 && gzf->size(0) == B && gzf->size(1) == M && gzf->device() == x.device(),
                "philtorch::lti_ss_backward: grad_zf must be (batch, M)");
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  const int dt = phs_dtype_of(x.scalar_type());
  Tensor Ac = A.contiguous(), xc = x.contiguous(), gc = gy.to(x.scalar_type()).contiguous();
  Tensor bc = Bm ? Bm->contiguous() : Tensor(), cc = Cm ? Cm->contiguous() : Tensor();
  Tensor dc = Dm ? Dm->contiguous() : Tensor(), zc = zi ? zi->contiguous() : Tensor();
  Tensor gzc = gzf ? gzf->to(x.scalar_type()).contiguous() : Tensor();
  Tensor gA = at::empty(A.sizes(), A.options());
  Tensor gB = Bm ? at::empty(Bm->sizes(), Bm->options()) : at::empty({0}, x.options());
  Tensor gC = Cm ? at::empty(Cm->sizes(), Cm->options()) : at::empty({0}, x.options());
  Tensor gD = Dm ? at::empty(Dm->sizes(), Dm->options()) : at::empty({0}, x.options());
  Tensor gzi = at::empty({B, M}, x.options());
  Tensor gx = at::empty_like(xc, at::MemoryFormat::Contiguous);
  if (B == 0) {
    gA.zero_(), gB.zero_(), gC.zero_(), gD.zero_();
    return {gA, gB, gC, gD, gzi, gx};
  }
  void *stream = stream_of(x);
  Tensor scratch = at::empty({int64_t(phs_lti_ss_bwd_scratch_size(dt, int(M), B, T))}, x.options().dtype(at::kByte));
  const Workspace ws = workspace_for(x, phs_lti_ss_workspace_size(dt, int(M), B, T), stream);
  check_status(phs_lti_ss_bwd_hs(dt, int(M), B, T, Ac.const_data_ptr(), A.dim() == 2 ? 1 : 0,
                              Bm ? bc.const_data_ptr() : nullptr, Bm && Bm->dim() == 1 ? 1 : 0,
                              Cm ? cc.const_data_ptr() : nullptr, Cm && Cm->dim() == 1 ? 1 : 0, int(out_idx),
                              Dm ? dc.const_data_ptr() : nullptr, Dm && Dm->numel() == 1 ? 1 : 0,
                              zi ? zc.const_data_ptr() : nullptr, xc.const_data_ptr(),
                              hs ? hc.const_data_ptr() : nullptr, gc.const_data_ptr(),
                              gzf ? gzc.const_data_ptr() : nullptr, gx.mutable_data_ptr(), gzi.mutable_data_ptr(),
                              gA.mutable_data_ptr(), Bm ? gB.mutable_data_ptr() : nullptr,
                              Cm ? gC.mutable_data_ptr() : nullptr, Dm ? gD.mutable_data_ptr() : nullptr,
                              reverse ? 1 : 0, scratch.mutable_data_ptr(), size_t(scratch.numel()), ws.ptr, ws.bytes,
                              stream),
               "lti_ss_backward");
  return {gA, gB, gC, gD, gzi, gx};
}

// Gradients of lfilter_ss w.r.t. (b, a, zi, x) (phs_lfilter_bwd): returns
// (grad_b, grad_a, grad_zi, grad_x) shaped like the inputs (grad_zi (batch,
// order) whether zi was given or not); grad_zf None is zero.  Replaces the
// autograd of the companion-form route (philtorch/lti/filtering.py:273-333).
std::vector<Tensor> lfilter_ss_backward_hip(const Tensor &b, const Tensor &a, const std::optional<Tensor> &zi,
                                            const Tensor &x, const Tensor &gy, const std::optional<Tensor> &gzf,
                                            int64_t form, bool reverse, const std::optional<Tensor> &hs) {
  (void)lfilter_ss_meta_check(b, a, zi, x, form);
  const int64_t B = x.size(0), T = x.size(1), nb = b.size(-1), na = a.size(-1);
  const int64_t M = std::max(nb - 1, na);
  check_states(hs, x, M, "lfilter_ss_backward");
  Tensor hc = hs ? hs->contiguous() : Tensor();
  TORCH_CHECK(gy.sizes() == x.sizes() && gy.device() == x.device(),
              "philtorch::lfilter_ss_backward: grad_y must have x's shape and device");
  if (gzf)
    TORCH_CHECK(gzf->dim() == 2 && gzf->size(0) == B && gzf->size(1) == M && gzf->device() == x.device(),
                "philtorch::lfilter_ss_backward: grad_zf must be (batch, order)");
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  const int dt = phs_dtype_of(x.scalar_type());
  Tensor bc = b.contiguous(), ac = a.contiguous(), xc = x.contiguous(), zc = zi ? zi->contiguous() : Tensor();
  Tensor gc = gy.to(x.scalar_type()).contiguous();
  Tensor gzc = gzf ? gzf->to(x.scalar_type()).contiguous() : Tensor();
  Tensor gb = at::empty(b.sizes(), b.options()), ga = at::empty(a.sizes(), a.options());
  Tensor gzi = at::empty({B, M}, x.options());
  Tensor gx = at::empty_like(xc, at::MemoryFormat::Contiguous);
  if (B == 0) {
    gb.zero_(), ga.zero_();
    return {gb, ga, gzi, gx};
  }
  void *stream = stream_of(x);
  Tensor scratch = at::empty({int64_t(phs_lti_ss_bwd_scratch_size(dt, int(M), B, T))}, x.options().dtype(at::kByte));
  const Workspace ws = workspace_for(x, phs_lti_ss_workspace_size(dt, int(M), B, T), stream);
  check_status(phs_lfilter_bwd_hs(dt, B, T, bc.const_data_ptr(), int(nb), ac.const_data_ptr(), int(na),
                               b.dim() == 1 ? 1 : 0, int(form), zi ? zc.const_data_ptr() : nullptr,
                               xc.const_data_ptr(), hs ? hc.const_data_ptr() : nullptr, gc.const_data_ptr(),
                               gzf ? gzc.const_data_ptr() : nullptr,
                               gx.mutable_data_ptr(), gzi.mutable_data_ptr(), gb.mutable_data_ptr(),
                               ga.mutable_data_ptr(), reverse ? 1 : 0, scratch.mutable_data_ptr(),
                               size_t(scratch.numel()), ws.ptr, ws.bytes, stream),
               "lfilter_ss_backward");
  return {gb, ga, gzi, gx};
}

// Single-input single-output LPV state space of order <= 4, fused
// (phs_lpv_ss_fwd; philtorch/lpv/ssm.py:337-581 for a 2D x): returns (y, zf).
// A (T, M, M) or (batch, T, M, M); B, C None or (1 | batch, 1 | T, M); D None
// or (1 | batch, 1 | T) (a size-1 axis is shared); zi None or (batch, M);
// out_idx selects the output state when C is None; reverse runs the model
// backwards in time (phs_lpv_ss_rev); transpose_A uses A[t]^T in place of
// A[t] (the adjoint model, read without a transposed copy).
// lpv_ss's argument checks (shared by its backward); returns M.
int64_t lpv_ss_meta_check(const Tensor &A, const std::optional<Tensor> &Bm, const std::optional<Tensor> &Cm,
                          const std::optional<Tensor> &Dm, const std::optional<Tensor> &zi, const Tensor &x,
                          int64_t out_idx) {
  TORCH_CHECK(x.dim() == 2, "philtorch::lpv_ss: x must be a 2D tensor (batch, time)");
  const int64_t B = x.size(0), T = x.size(1);
  TORCH_CHECK((A.dim() == 3 || A.dim() == 4) && A.size(-1) == A.size(-2) && A.size(-3) == T,
              "philtorch::lpv_ss: A must be (T, M, M) or (batch, T, M, M)");
  const int64_t M = A.size(-1);
  TORCH_CHECK(M >= 1 && M <= kMaxOrder, "philtorch::lpv_ss: state order 1 to ", kMaxOrder, ", got ", M);
  if (A.dim() == 4) TORCH_CHECK(A.size(0) == B, "philtorch::lpv_ss: a 4D A must have x's batch size");
  TORCH_CHECK(x.scalar_type() == at::kFloat || x.scalar_type() == at::kDouble,
              "philtorch::lpv_ss: float32 or float64 only, got ", x.scalar_type());
  TORCH_CHECK(x.is_cuda(), "philtorch::lpv_ss: philtorch_amd runs on HIP devices only (got ", x.device(), ")");
  auto same = [&](const Tensor &t, const char *what) {
    TORCH_CHECK(t.scalar_type() == x.scalar_type(), "philtorch::lpv_ss: ", what, " must have x's scalar type");
    TORCH_CHECK(t.device() == x.device(), "philtorch::lpv_ss: all tensors must be on the same device");
  };
  same(A, "A");
  auto vec_ok = [&](const Tensor &t) {
    return t.dim() == 3 && (t.size(0) == 1 || t.size(0) == B) && (t.size(1) == 1 || t.size(1) == T) &&
           t.size(2) == M;
  };
  if (Bm) {
    same(*Bm, "B");
    TORCH_CHECK(vec_ok(*Bm), "philtorch::lpv_ss: B must be (1 or batch, 1 or T, M)");
  }
  if (Cm) {
    same(*Cm, "C");
    TORCH_CHECK(vec_ok(*Cm), "philtorch::lpv_ss: C must be (1 or batch, 1 or T, M)");
  } else {
    TORCH_CHECK(out_idx >= 0 && out_idx < M, "philtorch::lpv_ss: out_idx must be in [0, ", M, ") when C is None");
  }
  if (Dm) {
    same(*Dm, "D");
    TORCH_CHECK(Dm->dim() == 2 && (Dm->size(0) == 1 || Dm->size(0) == B) && (Dm->size(1) == 1 || Dm->size(1) == T),
                "philtorch::lpv_ss: D must be (1 or batch, 1 or T)");
  }
  if (zi) {
    same(*zi, "zi");
    TORCH_CHECK(zi->dim() == 2 && zi->size(0) == B && zi->size(1) == M, "philtorch::lpv_ss: zi must be (batch, M)");
  }
  return M;
}

// element strides of a (rows, steps, width) lpv_ss operand with broadcast axes
int64_t lpv_row_stride(const Tensor &t, int64_t width) { return t.size(0) == 1 ? int64_t(0) : t.size(1) * width; }
int64_t lpv_t_stride(const Tensor &t, int64_t width) { return t.size(1) == 1 ? int64_t(0) : width; }

// keep_states: also the state before every step, hs (batch, T, M), written
// by the same pass (phs_lpv_ss_fwd_hs) for the coefficient backward.
std::tuple<Tensor, Tensor, Tensor> lpv_ss_impl(const Tensor &A, const std::optional<Tensor> &Bm,
                                               const std::optional<Tensor> &Cm, const std::optional<Tensor> &Dm,
                                               const std::optional<Tensor> &zi, const Tensor &x, int64_t out_idx,
                                               bool reverse, bool transpose_A, bool keep_states) {
  const int64_t M = lpv_ss_meta_check(A, Bm, Cm, Dm, zi, x, out_idx);
  const int64_t B = x.size(0), T = x.size(1);
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  const int dt = phs_dtype_of(x.scalar_type());
  Tensor Ac = A.contiguous(), xc = x.contiguous();
  Tensor bc = Bm ? Bm->contiguous() : Tensor(), cc = Cm ? Cm->contiguous() : Tensor();
  Tensor dc = Dm ? Dm->contiguous() : Tensor(), zc = zi ? zi->contiguous() : Tensor();
  Tensor y = at::empty_like(xc, at::MemoryFormat::Contiguous);
  Tensor zf = at::empty({B, M}, x.options());
  Tensor hs = at::empty({keep_states ? B : 0, keep_states ? T : 0, M}, x.options());
  if (B == 0) return {y, zf, hs};
  if (T == 0) {
    if (zi) zf.copy_(zc); else zf.zero_();
    return {y, zf, hs};
  }
  const auto rs = lpv_row_stride, ts = lpv_t_stride;
  void *stream = stream_of(x);
  const Workspace ws = workspace_for(x, phs_lpv_ss_workspace_size(dt, int(M), B, T), stream);
  const int A_flags = (A.dim() == 3 ? PHS_LPV_A_SHARED : 0) | (transpose_A ? PHS_LPV_A_TRANSPOSED : 0);
  const void *bp = Bm ? bc.const_data_ptr() : nullptr, *cp = Cm ? cc.const_data_ptr() : nullptr;
  const void *dp = Dm ? dc.const_data_ptr() : nullptr, *zp = zi ? zc.const_data_ptr() : nullptr;
  const int64_t brs = Bm ? rs(bc, M) : 0, bts = Bm ? ts(bc, M) : 0, crs = Cm ? rs(cc, M) : 0,
                cts = Cm ? ts(cc, M) : 0, drs = Dm ? rs(dc, 1) : 0, dts = Dm ? ts(dc, 1) : 0;
  if (keep_states)
    check_status(phs_lpv_ss_fwd_hs(dt, int(M), B, T, Ac.const_data_ptr(), A_flags, bp, brs, bts, cp, crs, cts,
                                   int(out_idx), dp, drs, dts, zp, xc.const_data_ptr(), y.mutable_data_ptr(),
                                   zf.mutable_data_ptr(), hs.mutable_data_ptr(), reverse ? 1 : 0, ws.ptr, ws.bytes,
                                   stream),
                 "lpv_ss_states");
  else
    check_status((reverse ? phs_lpv_ss_rev : phs_lpv_ss_fwd)(dt, int(M), B, T, Ac.const_data_ptr(), A_flags, bp, brs,
                                                             bts, cp, crs, cts, int(out_idx), dp, drs, dts, zp,
                                                             xc.const_data_ptr(), y.mutable_data_ptr(),
                                                             zf.mutable_data_ptr(), ws.ptr, ws.bytes, stream),
                 "lpv_ss");
  return {y, zf, hs};
}

std::tuple<Tensor, Tensor> lpv_ss_hip(const Tensor &A, const std::optional<Tensor> &Bm,
                                      const std::optional<Tensor> &Cm, const std::optional<Tensor> &Dm,
                                      const std::optional<Tensor> &zi, const Tensor &x, int64_t out_idx,
                                      bool reverse, bool transpose_A) {
  auto [y, zf, hs] = lpv_ss_impl(A, Bm, Cm, Dm, zi, x, out_idx, reverse, transpose_A, false);
  return {y, zf};
}

// lpv_ss that also returns hs (batch, T, M), the state before every step:
// what lpv_ss_backward would recompute for the coefficient gradients.
std::tuple<Tensor, Tensor, Tensor> lpv_ss_states_hip(const Tensor &A, const std::optional<Tensor> &Bm,
                                                     const std::optional<Tensor> &Cm,
                                                     const std::optional<Tensor> &Dm,
                                                     const std::optional<Tensor> &zi, const Tensor &x,
                                                     int64_t out_idx, bool reverse, bool transpose_A) {
  return lpv_ss_impl(A, Bm, Cm, Dm, zi, x, out_idx, reverse, transpose_A, true);
}

// Gradients of lpv_ss w.r.t. every input (phs_lpv_ss_bwd): returns (grad_A,
// grad_B, grad_C, grad_D, grad_zi, grad_x), each shaped like its input
// (summed over the axes the operand broadcasts; an absent operand's an empty
// tensor; grad_zi (batch, M) whether zi was given or not); grad_zf None is
// zero.  Replaces the autograd of the composed LPV state space
// (philtorch/lpv/ssm.py:337-581).
std::vector<Tensor> lpv_ss_backward_hip(const Tensor &A, const std::optional<Tensor> &Bm,
                                        const std::optional<Tensor> &Cm, const std::optional<Tensor> &Dm,
                                        const std::optional<Tensor> &zi, const Tensor &x, const Tensor &gy,
                                        const std::optional<Tensor> &gzf, int64_t out_idx, bool reverse,
                                        bool transpose_A, const std::optional<Tensor> &hs) {
  const int64_t M = lpv_ss_meta_check(A, Bm, Cm, Dm, zi, x, out_idx);
  const int64_t B = x.size(0), T = x.size(1);
  TORCH_CHECK(gy.sizes() == x.sizes() && gy.device() == x.device(),
              "philtorch::lpv_ss_backward: grad_y must have x's shape and device");
  if (hs)
    TORCH_CHECK(hs->dim() == 3 && hs->size(0) == B && hs->size(1) == T && hs->size(2) == M &&
                    hs->scalar_type() == x.scalar_type() && hs->device() == x.device(),
                "philtorch::lpv_ss_backward: hs must be the forward's states (batch, T, M)");
  Tensor hc = hs ? hs->contiguous() : Tensor();
  if (gzf)
    TORCH_CHECK(gzf->dim() == 2 && gzf->size(0) == B && gzf->size(1) == M && gzf->device() == x.device(),
                "philtorch::lpv_ss_backward: grad_zf must be (batch, M)");
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  const int dt = phs_dtype_of(x.scalar_type());
  Tensor Ac = A.contiguous(), xc = x.contiguous(), gc = gy.to(x.scalar_type()).contiguous();
  Tensor bc = Bm ? Bm->contiguous() : Tensor(), cc = Cm ? Cm->contiguous() : Tensor();
  Tensor dc = Dm ? Dm->contiguous() : Tensor(), zc = zi ? zi->contiguous() : Tensor();
  Tensor gzc = gzf ? gzf->to(x.scalar_type()).contiguous() : Tensor();
  Tensor gA = at::empty(A.sizes(), A.options());
  Tensor gB = Bm ? at::empty(Bm->sizes(), Bm->options()) : at::empty({0}, x.options());
  Tensor gC = Cm ? at::empty(Cm->sizes(), Cm->options()) : at::empty({0}, x.options());
  Tensor gD = Dm ? at::empty(Dm->sizes(), Dm->options()) : at::empty({0}, x.options());
  Tensor gzi = at::empty({B, M}, x.options());
  Tensor gx = at::empty_like(xc, at::MemoryFormat::Contiguous);
  if (B == 0) {
    gA.zero_(), gB.zero_(), gC.zero_(), gD.zero_();
    return {gA, gB, gC, gD, gzi, gx};
  }
  const auto rs = lpv_row_stride, ts = lpv_t_stride;
  auto tv_shared = [&](const std::optional<Tensor> &t, const Tensor &c, int64_t w) {
    return t && rs(c, w) == 0 && ts(c, w) != 0;
  };
  const int step_shared = (A.dim() == 3 ? PHS_LPV_GRAD_A : 0) | (tv_shared(Bm, bc, M) ? PHS_LPV_GRAD_B : 0) |
                          (tv_shared(Cm, cc, M) ? PHS_LPV_GRAD_C : 0) | (tv_shared(Dm, dc, 1) ? PHS_LPV_GRAD_D : 0);
  void *stream = stream_of(x);
  Tensor scratch =
      at::empty({int64_t(phs_lpv_ss_bwd_scratch_size(dt, int(M), B, T, step_shared))}, x.options().dtype(at::kByte));
  const Workspace ws = workspace_for(x, phs_lpv_ss_workspace_size(dt, int(M), B, T), stream);
  const int A_flags = (A.dim() == 3 ? PHS_LPV_A_SHARED : 0) | (transpose_A ? PHS_LPV_A_TRANSPOSED : 0);
  check_status(phs_lpv_ss_bwd_hs(dt, int(M), B, T, Ac.const_data_ptr(), A_flags, Bm ? bc.const_data_ptr() : nullptr,
                              Bm ? rs(bc, M) : 0, Bm ? ts(bc, M) : 0, Cm ? cc.const_data_ptr() : nullptr,
                              Cm ? rs(cc, M) : 0, Cm ? ts(cc, M) : 0, int(out_idx),
                              Dm ? dc.const_data_ptr() : nullptr, Dm ? rs(dc, 1) : 0, Dm ? ts(dc, 1) : 0,
                              zi ? zc.const_data_ptr() : nullptr, xc.const_data_ptr(),
                              hs ? hc.const_data_ptr() : nullptr, gc.const_data_ptr(),
                              gzf ? gzc.const_data_ptr() : nullptr, gx.mutable_data_ptr(), gzi.mutable_data_ptr(),
                              gA.mutable_data_ptr(), Bm ? gB.mutable_data_ptr() : nullptr,
                              Cm ? gC.mutable_data_ptr() : nullptr, Dm ? gD.mutable_data_ptr() : nullptr,
                              reverse ? 1 : 0, scratch.mutable_data_ptr(), size_t(scratch.numel()), ws.ptr, ws.bytes,
                              stream),
               "lpv_ss_backward");
  return {gA, gB, gC, gD, gzi, gx};
}

// Multi-input, multi-output LPV state space (time-varying A) of order <= 4
// with 1-4 inputs and outputs per step, B, C, D constant in time, fused
// (phs_lpv_mimo_ss; philtorch/lpv/ssm.py:337-581 for a 3D x or matrix
// B, C, D): returns (y, zf).  x (batch, T, F); A (T, M, M) or
// (batch, T, M, M); B (M, F) or (batch, M, F); C (P, M) or (batch, P, M);
// D None, (P, F) or (batch, P, F); zi None or (batch, M); y (batch, T, P).
// reverse runs the model backwards in time; transpose_A uses A[t]^T (the
// adjoint model, read without a transposed copy).
std::tuple<Tensor, Tensor, Tensor> lpv_mimo_ss_impl(const Tensor &A, const Tensor &Bm, const Tensor &Cm,
                                                    const std::optional<Tensor> &Dm,
                                                    const std::optional<Tensor> &zi, const Tensor &x, bool reverse,
                                                    bool transpose_A, bool keep_states) {
  TORCH_CHECK(x.dim() == 3, "philtorch::lpv_mimo_ss: x must be a 3D tensor (batch, time, features)");
  const int64_t B = x.size(0), T = x.size(1), F = x.size(2);
  TORCH_CHECK((A.dim() == 3 || A.dim() == 4) && A.size(-1) == A.size(-2) && A.size(-3) == T,
              "philtorch::lpv_mimo_ss: A must be (T, M, M) or (batch, T, M, M)");
  if (A.dim() == 4) TORCH_CHECK(A.size(0) == B, "philtorch::lpv_mimo_ss: a 4D A must have x's batch size");
  const int64_t M = A.size(-1);
  TORCH_CHECK(M >= 1 && M <= kMaxOrder, "philtorch::lpv_mimo_ss: state order 1 to ", kMaxOrder, ", got ", M);
  TORCH_CHECK(F >= 1 && F <= 4, "philtorch::lpv_mimo_ss: 1 to 4 input features, got ", F);
  TORCH_CHECK(Cm.dim() == 2 || Cm.dim() == 3, "philtorch::lpv_mimo_ss: C must be (P, M) or (batch, P, M)");
  const int64_t P = Cm.size(-2);
  TORCH_CHECK(P >= 1 && P <= 4, "philtorch::lpv_mimo_ss: 1 to 4 outputs, got ", P);
  TORCH_CHECK(x.scalar_type() == at::kFloat || x.scalar_type() == at::kDouble,
              "philtorch::lpv_mimo_ss: float32 or float64 only, got ", x.scalar_type());
  TORCH_CHECK(x.is_cuda(), "philtorch::lpv_mimo_ss: philtorch_amd runs on HIP devices only (got ", x.device(), ")");
  TORCH_CHECK(A.scalar_type() == x.scalar_type() && A.device() == x.device(),
              "philtorch::lpv_mimo_ss: A must have x's scalar type and device");
  auto check = [&](const Tensor &t, const char *what, int64_t r, int64_t c) {
    TORCH_CHECK(t.scalar_type() == x.scalar_type(), "philtorch::lpv_mimo_ss: ", what, " must have x's scalar type");
    TORCH_CHECK(t.device() == x.device(), "philtorch::lpv_mimo_ss: all tensors must be on the same device");
    TORCH_CHECK((t.dim() == 2 || (t.dim() == 3 && t.size(0) == B)) && t.size(-2) == r && t.size(-1) == c,
                "philtorch::lpv_mimo_ss: ", what, " must be (", r, ", ", c, ") or (batch, ", r, ", ", c, "), got ",
                t.sizes());
  };
  check(Bm, "B", M, F);
  check(Cm, "C", P, M);
  if (Dm) check(*Dm, "D", P, F);
  if (zi) {
    TORCH_CHECK(zi->scalar_type() == x.scalar_type() && zi->device() == x.device(),
                "philtorch::lpv_mimo_ss: zi must have x's scalar type and device");
    TORCH_CHECK(zi->dim() == 2 && zi->size(0) == B && zi->size(1) == M,
                "philtorch::lpv_mimo_ss: zi must be (batch, M)");
  }
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  const int dt = phs_dtype_of(x.scalar_type());
  Tensor Ac = A.contiguous(), bc = Bm.contiguous(), cc = Cm.contiguous(), xc = x.contiguous();
  Tensor dc = Dm ? Dm->contiguous() : Tensor(), zc = zi ? zi->contiguous() : Tensor();
  Tensor y = at::empty({B, T, P}, x.options());
  Tensor zf = at::empty({B, M}, x.options());
  Tensor hs = at::empty({keep_states ? B : 0, keep_states ? T : 0, M}, x.options());
  if (keep_states)
    TORCH_CHECK(P + M <= 4, "philtorch::lpv_mimo_ss_states: outputs plus states at most 4 per step, got ", P, " + ", M);
  if (B == 0) return {y, zf, hs};
  if (T == 0) {
    if (zi) zf.copy_(zc); else zf.zero_();
    return {y, zf, hs};
  }
  const int A_flags = (A.dim() == 3 ? PHS_LPV_A_SHARED : 0) | (transpose_A ? PHS_LPV_A_TRANSPOSED : 0);
  const int shared = (Bm.dim() == 2 ? PHS_MIMO_B_SHARED : 0) | (Cm.dim() == 2 ? PHS_MIMO_C_SHARED : 0) |
                     (Dm && Dm->dim() == 2 ? PHS_MIMO_D_SHARED : 0);
  void *stream = stream_of(x);
  const Workspace ws = workspace_for(x, phs_lpv_mimo_ss_workspace_size(dt, int(M), B, T), stream);
  check_status(phs_lpv_mimo_ss_hs(dt, int(M), int(F), int(P), B, T, Ac.const_data_ptr(), A_flags,
                                  bc.const_data_ptr(), cc.const_data_ptr(), Dm ? dc.const_data_ptr() : nullptr, shared,
                                  zi ? zc.const_data_ptr() : nullptr, xc.const_data_ptr(), y.mutable_data_ptr(),
                                  zf.mutable_data_ptr(), keep_states ? hs.mutable_data_ptr() : nullptr,
                                  reverse ? 1 : 0, ws.ptr, ws.bytes, stream),
               "lpv_mimo_ss");
  return {y, zf, hs};
}

std::tuple<Tensor, Tensor> lpv_mimo_ss_hip(const Tensor &A, const Tensor &Bm, const Tensor &Cm,
                                           const std::optional<Tensor> &Dm, const std::optional<Tensor> &zi,
                                           const Tensor &x, bool reverse, bool transpose_A) {
  auto [y, zf, hs] = lpv_mimo_ss_impl(A, Bm, Cm, Dm, zi, x, reverse, transpose_A, false);
  return {y, zf};
}

// lpv_mimo_ss that also returns hs (batch, T, M), the state before every
// step (the states the coefficient gradients read), from the same pass.
std::tuple<Tensor, Tensor, Tensor> lpv_mimo_ss_states_hip(const Tensor &A, const Tensor &Bm, const Tensor &Cm,
                                                          const std::optional<Tensor> &Dm,
                                                          const std::optional<Tensor> &zi, const Tensor &x,
                                                          bool reverse, bool transpose_A) {
  return lpv_mimo_ss_impl(A, Bm, Cm, Dm, zi, x, reverse, transpose_A, true);
}

// The coefficient gradients of mimo_ss summed over time in one pass
// (phs_mimo_ss_grad_sums): lam, hs (batch, T, M) (None where no wanted
// output reads them), x (batch, T, F), g (batch, T, P); `want` and `shared`
// bit i for A, B, C, D.  Returns [gA, gB, gC, gD], each (batch or 1, rows,
// cols) as its bit in `shared` says, an empty tensor where not wanted;
// with PHS_MIMO_A_STEPS (and _T) in `shared`, gA is (batch, T, M, M), the
// per-step product lam[t] h[t]^T (transposed).  want bit 4: a fifth tensor,
// the input's gradient (batch, T, F) = Bm^T lam[t] + Dm^T g[t] from the
// model's Bm (M, F) / (batch, M, F) and Dm None / (P, F) / (batch, P, F).
std::vector<Tensor> mimo_ss_grad_sums_hip(const std::optional<Tensor> &lam, const std::optional<Tensor> &hs,
                                          const Tensor &x, const Tensor &g, int64_t shared, int64_t want,
                                          const std::optional<Tensor> &Bm, const std::optional<Tensor> &Dm) {
  TORCH_CHECK(x.dim() == 3 && g.dim() == 3 && g.size(0) == x.size(0) && g.size(1) == x.size(1),
              "philtorch::mimo_ss_grad_sums: x and g must be (batch, T, F) and (batch, T, P)");
  TORCH_CHECK((want & ~31) == 0 && (shared & ~63) == 0,
              "philtorch::mimo_ss_grad_sums: want is a 5-bit mask, shared a 6-bit one");
  const bool want_gx = want & 16;
  TORCH_CHECK(!want_gx || (lam && Bm), "philtorch::mimo_ss_grad_sums: the input's gradient needs lam and Bm");
  const bool steps = shared & PHS_MIMO_A_STEPS;
  TORCH_CHECK(!(steps && (shared & PHS_MIMO_A_SHARED)) && (steps || !(shared & PHS_MIMO_A_STEPS_T)),
              "philtorch::mimo_ss_grad_sums: A per step is neither shared nor transposed without A_STEPS");
  const int64_t B = x.size(0), T = x.size(1), F = x.size(2), P = g.size(2);
  const bool need_l = want & 3, need_h = want & 5;
  TORCH_CHECK(!need_l || lam, "philtorch::mimo_ss_grad_sums: gradients of A or B need lam");
  TORCH_CHECK(!need_h || hs, "philtorch::mimo_ss_grad_sums: gradients of A or C need hs");
  const Tensor &ref = lam ? *lam : *hs;
  const int64_t M = (lam || hs) ? ref.size(2) : 1;
  for (const Tensor *t : {lam ? &*lam : nullptr, hs ? &*hs : nullptr, &x, &g}) {
    if (!t) continue;
    TORCH_CHECK(t->dim() == 3 && t->size(0) == B && t->size(1) == T, "philtorch::mimo_ss_grad_sums: (batch, T, n) operands");
    TORCH_CHECK(t->scalar_type() == x.scalar_type() && t->device() == x.device(),
                "philtorch::mimo_ss_grad_sums: one dtype and device");
  }
  if (lam) TORCH_CHECK(lam->size(2) == M, "philtorch::mimo_ss_grad_sums: lam and hs must both have M states");
  if (hs) TORCH_CHECK(hs->size(2) == M, "philtorch::mimo_ss_grad_sums: lam and hs must both have M states");
  Tensor bc, dc;
  if (want_gx) {
    auto model = [&](const Tensor &t, int64_t r, int bit, const char *what) {
      TORCH_CHECK(t.scalar_type() == x.scalar_type() && t.device() == x.device(),
                  "philtorch::mimo_ss_grad_sums: ", what, " must have x's dtype and device");
      const bool sh = (shared >> bit) & 1;
      TORCH_CHECK(t.dim() == (sh ? 2 : 3) && (sh || t.size(0) == B) && t.size(-2) == r && t.size(-1) == F,
                  "philtorch::mimo_ss_grad_sums: ", what, " must be (", r, ", ", F, "), or per row as its shared bit says");
      return t.contiguous();
    };
    bc = model(*Bm, M, 1, "Bm");
    if (Dm) dc = model(*Dm, P, 3, "Dm");
  }
  TORCH_CHECK(x.scalar_type() == at::kFloat || x.scalar_type() == at::kDouble,
              "philtorch::mimo_ss_grad_sums: float32 or float64 only");
  TORCH_CHECK(x.is_cuda(), "philtorch::mimo_ss_grad_sums: HIP tensors only");
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  const int dt = phs_dtype_of(x.scalar_type());
  Tensor lc = lam ? lam->contiguous() : Tensor(), hc = hs ? hs->contiguous() : Tensor();
  Tensor xc = x.contiguous(), gc = g.contiguous();
  const int64_t rows[4] = {M, M, P, P}, cols[4] = {M, F, M, F};
  std::vector<Tensor> out(want_gx ? 5 : 4);
  if (want_gx) out[4] = at::empty({B, T, F}, x.options());
  for (int p = 0; p < 4; ++p) {
    if (p == 0 && steps && (want & 1)) {
      out[p] = at::empty({B, T, M, M}, x.options());
    } else if ((want >> p) & 1) {
      out[p] = at::empty({((shared >> p) & 1) ? int64_t(1) : B, rows[p], cols[p]}, x.options());
      if (B == 0 || T == 0) out[p].zero_();
    } else {
      out[p] = at::empty({0}, x.options());
    }
  }
  if (B == 0 || T == 0 || want == 0) return out;
  Tensor scratch = at::empty({int64_t(std::max<size_t>(phs_mimo_ss_grad_sums_scratch_size(dt, B, T), 8))},
                             x.options().dtype(at::kByte));
  auto ptr = [&](int p) { return ((want >> p) & 1) ? out[p].mutable_data_ptr() : nullptr; };
  check_status(phs_mimo_ss_grad_sums(dt, int(M), int(F), int(P), B, T, lam ? lc.const_data_ptr() : nullptr,
                                     hs ? hc.const_data_ptr() : nullptr, xc.const_data_ptr(), gc.const_data_ptr(),
                                     want_gx ? bc.const_data_ptr() : nullptr,
                                     want_gx && Dm ? dc.const_data_ptr() : nullptr, int(shared), ptr(0), ptr(1),
                                     ptr(2), ptr(3), ptr(4), scratch.mutable_data_ptr(), size_t(scratch.numel()),
                                     stream_of(x)),
               "mimo_ss_grad_sums");
  return out;
}

// Multi-input, multi-output LTI state space of order <= 4 with 1-4 inputs and
// 1-4 outputs per step, fused (phs_mimo_ss_fwd; philtorch/lti/ssm.py:386-589
// for a 3D x or matrix-valued B, C, D): returns (y, zf).  x (batch, T, F);
// A (M, M) or (batch, M, M); B (M, F) or (batch, M, F); C (P, M) or
// (batch, P, M); D None, (P, F) or (batch, P, F); zi None or (batch, M);
// y (batch, T, P).  reverse runs the model backwards in time
// (phs_mimo_ss_rev), the form of its adjoint.
std::tuple<Tensor, Tensor> mimo_ss_hip(const Tensor &A, const Tensor &Bm, const Tensor &Cm,
                                       const std::optional<Tensor> &Dm, const std::optional<Tensor> &zi,
                                       const Tensor &x, bool reverse) {
  TORCH_CHECK(x.dim() == 3, "philtorch::mimo_ss: x must be a 3D tensor (batch, time, features)");
  const int64_t B = x.size(0), T = x.size(1), F = x.size(2);
  TORCH_CHECK((A.dim() == 2 || A.dim() == 3) && A.size(-1) == A.size(-2),
              "philtorch::mimo_ss: A must be (M, M) or (batch, M, M)");
  const int64_t M = A.size(-1);
  TORCH_CHECK(M >= 1 && M <= kMaxOrder, "philtorch::mimo_ss: state order 1 to ", kMaxOrder, ", got ", M);
  TORCH_CHECK(F >= 1 && F <= 4, "philtorch::mimo_ss: 1 to 4 input features, got ", F);
  TORCH_CHECK(Cm.dim() == 2 || Cm.dim() == 3, "philtorch::mimo_ss: C must be (P, M) or (batch, P, M)");
  const int64_t P = Cm.size(-2);
  TORCH_CHECK(P >= 1 && P <= 4, "philtorch::mimo_ss: 1 to 4 outputs, got ", P);
  TORCH_CHECK(x.scalar_type() == at::kFloat || x.scalar_type() == at::kDouble,
              "philtorch::mimo_ss: float32 or float64 only, got ", x.scalar_type());
  TORCH_CHECK(x.is_cuda(), "philtorch::mimo_ss: philtorch_amd runs on HIP devices only (got ", x.device(), ")");
  auto check = [&](const Tensor &t, const char *what, int64_t r, int64_t c) {
    TORCH_CHECK(t.scalar_type() == x.scalar_type(), "philtorch::mimo_ss: ", what, " must have x's scalar type");
    TORCH_CHECK(t.device() == x.device(), "philtorch::mimo_ss: all tensors must be on the same device");
    TORCH_CHECK((t.dim() == 2 || (t.dim() == 3 && t.size(0) == B)) && t.size(-2) == r && t.size(-1) == c,
                "philtorch::mimo_ss: ", what, " must be (", r, ", ", c, ") or (batch, ", r, ", ", c, "), got ",
                t.sizes());
  };
  check(A, "A", M, M);
  check(Bm, "B", M, F);
  check(Cm, "C", P, M);
  if (Dm) check(*Dm, "D", P, F);
  if (zi) {
    TORCH_CHECK(zi->scalar_type() == x.scalar_type() && zi->device() == x.device(),
                "philtorch::mimo_ss: zi must have x's scalar type and device");
    TORCH_CHECK(zi->dim() == 2 && zi->size(0) == B && zi->size(1) == M, "philtorch::mimo_ss: zi must be (batch, M)");
  }
  const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
  const int dt = phs_dtype_of(x.scalar_type());
  Tensor Ac = A.contiguous(), bc = Bm.contiguous(), cc = Cm.contiguous(), xc = x.contiguous();
  Tensor dc = Dm ? Dm->contiguous() : Tensor(), zc = zi ? zi->contiguous() : Tensor();
  Tensor y = at::empty({B, T, P}, x.options());
  Tensor zf = at::empty({B, M}, x.options());
  if (B == 0) return {y, zf};
  if (T == 0) {
    if (zi) zf.copy_(zc); else zf.zero_();
    return {y, zf};
  }
  const int shared = (A.dim() == 2 ? PHS_MIMO_A_SHARED : 0) | (Bm.dim() == 2 ? PHS_MIMO_B_SHARED : 0) |
                     (Cm.dim() == 2 ? PHS_MIMO_C_SHARED : 0) | (Dm && Dm->dim() == 2 ? PHS_MIMO_D_SHARED : 0);
  void *stream = stream_of(x);
  const Workspace ws = workspace_for(x, phs_mimo_ss_workspace_size(dt, int(M), B, T), stream);
  check_status((reverse ? phs_mimo_ss_rev : phs_mimo_ss_fwd)(
                   dt, int(M), int(F), int(P), B, T, Ac.const_data_ptr(), bc.const_data_ptr(), cc.const_data_ptr(),
                   Dm ? dc.const_data_ptr() : nullptr, shared, zi ? zc.const_data_ptr() : nullptr,
                   xc.const_data_ptr(), y.mutable_data_ptr(), zf.mutable_data_ptr(), ws.ptr, ws.bytes, stream),
               "mimo_ss");
  return {y, zf};
}

// ------------------------------------------------------------ CPU key
// The reference's CPU extension registers its ops for the CPU key; these
// run phs_cpu.hpp on contiguous copies, in parallel over rows (torch's
// intra-op thread pool), serially in time.  Half and bfloat16 compute in their
// own type, rounding after every operation, as the reference's CPU loops do
// (its AT_DISPATCH ..._AND2/AND3(kHalf, kBFloat16) kernels); the backward's
// sums over steps or rows accumulate them in float.
template <class F>
void parallel_rows(int64_t n, F &&f) {
  at::parallel_for(0, n, 1, [&](int64_t begin, int64_t end) {
    for (int64_t i = begin; i < end; ++i) f(i);
  });
}

void check_cpu(const char *op, const Tensor &x) {
  TORCH_CHECK(x.is_cpu(), "philtorch::", op, ": CPU kernel called with a ", x.device(), " tensor");
}

// y = scan(A, zi, x); x [B, T] or [B, T, M]; A laid out as L says.
Tensor cpu_fwd(const Tensor &A, const Tensor &zi, const Tensor &x, phs_cpu::Layout L) {
  Tensor Ac = A.contiguous(), zc = zi.contiguous(), xc = x.contiguous();
  Tensor y = at::empty_like(xc, at::MemoryFormat::Contiguous);
  if (L.B == 0 || L.T == 0) return y;
  AT_DISPATCH_FLOATING_AND_COMPLEX_TYPES_AND3(at::kLong, at::kHalf, at::kBFloat16, x.scalar_type(), "philtorch_cpu_fwd", [&] {
    phs_cpu::scan_fwd<scalar_t>(L, Ac.const_data_ptr<scalar_t>(), zc.const_data_ptr<scalar_t>(),
                                xc.const_data_ptr<scalar_t>(), y.mutable_data_ptr<scalar_t>(),
                                [](int64_t n, auto &&f) { parallel_rows(n, f); });
  });
  return y;
}

// (grad_A in A's shape, grad_zi, grad_x) of cpu_fwd for upstream grad gy.
Triple cpu_bwd(const Tensor &A, const Tensor &zi, const Tensor &y, const Tensor &gy, phs_cpu::Layout L) {
  Tensor Ac = A.contiguous(), zc = zi.contiguous(), yc = y.contiguous(), gc = gy.contiguous();
  Tensor gA = at::empty(A.sizes(), A.options());
  Tensor gzi = at::empty(zi.sizes(), zi.options());
  Tensor gx = at::empty(y.sizes(), y.options());
  if (L.B == 0 || L.T == 0) return {gA.zero_(), gzi.zero_(), gx.zero_()};
  AT_DISPATCH_FLOATING_AND_COMPLEX_TYPES_AND3(at::kLong, at::kHalf, at::kBFloat16, y.scalar_type(), "philtorch_cpu_bwd", [&] {
    phs_cpu::scan_bwd<scalar_t>(L, Ac.const_data_ptr<scalar_t>(), zc.const_data_ptr<scalar_t>(),
                                yc.const_data_ptr<scalar_t>(), gc.const_data_ptr<scalar_t>(),
                                gx.mutable_data_ptr<scalar_t>(), gA.mutable_data_ptr<scalar_t>(),
                                gzi.mutable_data_ptr<scalar_t>(),
                                [](int64_t n, auto &&f) { parallel_rows(n, f); });
  });
  return {gA, gzi, gx};
}

Tensor recur_cpu(const Tensor &A, const Tensor &zi, const Tensor &x) {
  check_common("recur", A, zi, x);
  check_recur(A, zi, x);
  check_cpu("recur", x);
  const int64_t B = x.size(0), T = x.size(1);
  return cpu_fwd(A, zi, x, {B, T, 1, A.dim() == 1 ? 0 : T, 1, false});
}

Triple recur_backward_cpu(const Tensor &A, const Tensor &zi, const Tensor &y, const Tensor &gy) {
  check_common("recur_backward", A, zi, y);
  check_recur(A, zi, y);
  check_cpu("recur_backward", y);
  TORCH_CHECK(gy.sizes() == y.sizes(), "grad_y must have y's shape");
  const int64_t B = y.size(0), T = y.size(1);
  return cpu_bwd(A, zi, y, gy.to(y.scalar_type()), {B, T, 1, A.dim() == 1 ? 0 : T, 1, false});
}

Tensor recurN_cpu(const Tensor &A, const Tensor &zi, const Tensor &x) {
  check_common("recurN", A, zi, x);
  check_recurN(A, zi, x);
  check_cpu("recurN", x);
  const int64_t B = x.size(0), T = x.size(1), M = A.size(-1);
  return cpu_fwd(A, zi, x, {B, T, M, A.dim() == 3 ? 0 : T * M * M, M * M, false});
}

Tensor recur2_cpu(const Tensor &A, const Tensor &zi, const Tensor &x) {
  TORCH_CHECK(A.dim() >= 2 && A.size(-1) == 2 && A.size(-2) == 2, "A must be square.");
  return recurN_cpu(A, zi, x);
}

Triple recurN_backward_cpu(const Tensor &A, const Tensor &zi, const Tensor &y, const Tensor &gy) {
  check_common("recurN_backward", A, zi, y);
  check_recurN(A, zi, y);
  check_cpu("recurN_backward", y);
  TORCH_CHECK(gy.sizes() == y.sizes(), "grad_y must have y's shape");
  const int64_t B = y.size(0), T = y.size(1), M = A.size(-1);
  return cpu_bwd(A, zi, y, gy.to(y.scalar_type()), {B, T, M, A.dim() == 3 ? 0 : T * M * M, M * M, false});
}

Tensor lti_recur_cpu(const Tensor &A, const Tensor &zi, const Tensor &x) {
  check_common("lti_recur", A, zi, x);
  check_lti_recur(A, zi, x);
  check_cpu("lti_recur", x);
  const int64_t B = x.size(0), T = x.size(1);
  return cpu_fwd(A, zi, x, {B, T, 1, lti_shared(A, x) ? 0 : 1, 0, true});
}

Triple lti_recur_backward_cpu(const Tensor &A, const Tensor &zi, const Tensor &y, const Tensor &gy) {
  check_common("lti_recur_backward", A, zi, y);
  check_lti_recur(A, zi, y);
  check_cpu("lti_recur_backward", y);
  TORCH_CHECK(gy.sizes() == y.sizes(), "grad_y must have y's shape");
  const int64_t B = y.size(0), T = y.size(1);
  return cpu_bwd(A, zi, y, gy.to(y.scalar_type()), {B, T, 1, lti_shared(A, y) ? 0 : 1, 0, true});
}

Tensor lti_recurN_cpu(const Tensor &A, const Tensor &zi, const Tensor &x) {
  check_common("lti_recurN", A, zi, x);
  check_lti_recurN(A, zi, x);
  check_cpu("lti_recurN", x);
  const int64_t B = x.size(0), T = x.size(1), M = A.size(-1);
  return cpu_fwd(A, zi, x, {B, T, M, A.dim() == 2 ? 0 : M * M, 0, false});
}

Tensor lti_recur2_cpu(const Tensor &A, const Tensor &zi, const Tensor &x) {
  TORCH_CHECK(A.dim() >= 2 && A.size(-1) == 2 && A.size(-2) == 2, "A must be square.");
  return lti_recurN_cpu(A, zi, x);
}

Triple lti_recurN_backward_cpu(const Tensor &A, const Tensor &zi, const Tensor &y, const Tensor &gy) {
  check_common("lti_recurN_backward", A, zi, y);
  check_lti_recurN(A, zi, y);
  check_cpu("lti_recurN_backward", y);
  TORCH_CHECK(gy.sizes() == y.sizes(), "grad_y must have y's shape");
  const int64_t B = y.size(0), T = y.size(1), M = A.size(-1);
  return cpu_bwd(A, zi, y, gy.to(y.scalar_type()), {B, T, M, A.dim() == 2 ? 0 : M * M, 0, false});
}

}  // namespace

TORCH_LIBRARY(philtorch, m) {
  // the reference's five schemas, philtorch/csrc/host_recur2.cpp:164-170
  m.def("recur2(Tensor A, Tensor zi, Tensor x) -> Tensor", {at::Tag::pt2_compliant_tag});
  m.def("recurN(Tensor A, Tensor zi, Tensor x) -> Tensor", {at::Tag::pt2_compliant_tag});
  m.def("lti_recur2(Tensor A, Tensor zi, Tensor x) -> Tensor", {at::Tag::pt2_compliant_tag});
  m.def("lti_recurN(Tensor A, Tensor zi, Tensor x) -> Tensor", {at::Tag::pt2_compliant_tag});
  m.def("lti_recur(Tensor A, Tensor zi, Tensor x) -> Tensor", {at::Tag::pt2_compliant_tag});
  // new: the LPV scalar scan behind lpv.linear_recurrence (A [B,T] or [T])
  m.def("recur(Tensor A, Tensor zi, Tensor x) -> Tensor", {at::Tag::pt2_compliant_tag});
  // new: fused adjoint passes returning (grad_A, grad_zi, grad_x)
  m.def("recur_backward(Tensor A, Tensor zi, Tensor y, Tensor grad_y) -> (Tensor, Tensor, Tensor)",
        {at::Tag::pt2_compliant_tag});
  m.def("recurN_backward(Tensor A, Tensor zi, Tensor y, Tensor grad_y) -> (Tensor, Tensor, Tensor)",
        {at::Tag::pt2_compliant_tag});
  m.def("lti_recur_backward(Tensor A, Tensor zi, Tensor y, Tensor grad_y) -> (Tensor, Tensor, Tensor)",
        {at::Tag::pt2_compliant_tag});
  m.def("lti_recurN_backward(Tensor A, Tensor zi, Tensor y, Tensor grad_y) -> (Tensor, Tensor, Tensor)",
        {at::Tag::pt2_compliant_tag});
  // new: fused cascade of second-order sections, returning (y, zf, ckpt), and
  // its backward returning (grad_x, grad_sos, grad_zi)
  m.def("sosfilt(Tensor sos, Tensor? zi, Tensor x) -> (Tensor, Tensor, Tensor)", {at::Tag::pt2_compliant_tag});
  m.def("sosfilt_backward(Tensor sos, Tensor x, Tensor ckpt, Tensor grad_y, Tensor? grad_zf, bool need_sos)"
        " -> (Tensor, Tensor, Tensor)",
        {at::Tag::pt2_compliant_tag});
  // new: one biquad on the cascade kernel from lfilter's b and a, and its backward
  m.def("biquad(Tensor b, Tensor a, Tensor? zi, Tensor x) -> (Tensor, Tensor, Tensor)", {at::Tag::pt2_compliant_tag});
  m.def("biquad_backward(Tensor b, Tensor a, Tensor x, Tensor ckpt, Tensor grad_y, Tensor? grad_zf, bool need_coef)"
        " -> Tensor[]",
        {at::Tag::pt2_compliant_tag});
  // new: the same with b and a as columns of coefficient tables (col -1: b or a itself);
  // the backward's coefficient gradients are the whole tables'
  m.def("biquad_cols(Tensor bt, int b_col, Tensor at, int a_col, Tensor? zi, Tensor x) -> (Tensor, Tensor, Tensor)",
        {at::Tag::pt2_compliant_tag});
  m.def("biquad_cols_backward(Tensor bt, int b_col, Tensor at, int a_col, Tensor x, Tensor ckpt, Tensor grad_y, "
        "Tensor? grad_zf, bool need_coef) -> Tensor[]",
        {at::Tag::pt2_compliant_tag});
  // new: zero-phase filtering, filters of second order at most (forward only)
  m.def("filtfilt(Tensor b, Tensor a, Tensor x, int padmode, int padlen) -> Tensor", {at::Tag::pt2_compliant_tag});
  m.def("filtfilt_backward(Tensor b, Tensor a, Tensor x, Tensor grad_y, int padmode, int padlen, bool need_coef, "
        "Tensor? mid=None, Tensor? h1=None, Tensor? h2=None) -> Tensor[]",
        {at::Tag::pt2_compliant_tag});
  m.def("filtfilt_states(Tensor b, Tensor a, Tensor x, int padmode, int padlen) -> (Tensor, Tensor, Tensor, Tensor)",
        {at::Tag::pt2_compliant_tag});
  // new: single-input single-output LTI state space of order <= 4, fused: (y, zf)
  m.def("lti_ss(Tensor A, Tensor? B, Tensor? C, Tensor? D, Tensor? zi, Tensor x, int out_idx, bool reverse=False) -> (Tensor, Tensor)",
        {at::Tag::pt2_compliant_tag});
  // new: lfilter of order <= 4 from b and a (companion model built in the kernel): (y, zf)
  m.def("lfilter_ss(Tensor b, Tensor a, Tensor? zi, Tensor x, int form, bool reverse=False) -> (Tensor, Tensor)",
        {at::Tag::pt2_compliant_tag});
  // new: their fused gradients w.r.t. every input (coefficients included)
  m.def("lti_ss_backward(Tensor A, Tensor? B, Tensor? C, Tensor? D, Tensor? zi, Tensor x, Tensor grad_y, "
        "Tensor? grad_zf, int out_idx, bool reverse=False, Tensor? hs=None) -> Tensor[]",
        {at::Tag::pt2_compliant_tag});
  m.def("lfilter_ss_backward(Tensor b, Tensor a, Tensor? zi, Tensor x, Tensor grad_y, Tensor? grad_zf, int form, "
        "bool reverse=False, Tensor? hs=None) -> Tensor[]",
        {at::Tag::pt2_compliant_tag});
  // new: the forwards that also return their states, for the coefficient backward
  m.def("lti_ss_states(Tensor A, Tensor? B, Tensor? C, Tensor? D, Tensor? zi, Tensor x, int out_idx, "
        "bool reverse=False) -> (Tensor, Tensor, Tensor)",
        {at::Tag::pt2_compliant_tag});
  m.def("lfilter_ss_states(Tensor b, Tensor a, Tensor? zi, Tensor x, int form, bool reverse=False) -> "
        "(Tensor, Tensor, Tensor)",
        {at::Tag::pt2_compliant_tag});
  m.def("lpv_ss(Tensor A, Tensor? B, Tensor? C, Tensor? D, Tensor? zi, Tensor x, int out_idx, bool reverse=False, "
        "bool transpose_A=False) -> (Tensor, Tensor)",
        {at::Tag::pt2_compliant_tag});
  m.def("lpv_ss_backward(Tensor A, Tensor? B, Tensor? C, Tensor? D, Tensor? zi, Tensor x, Tensor grad_y, "
        "Tensor? grad_zf, int out_idx, bool reverse=False, bool transpose_A=False, Tensor? hs=None) -> Tensor[]",
        {at::Tag::pt2_compliant_tag});
  m.def("lpv_ss_states(Tensor A, Tensor? B, Tensor? C, Tensor? D, Tensor? zi, Tensor x, int out_idx, "
        "bool reverse=False, bool transpose_A=False) -> (Tensor, Tensor, Tensor)",
        {at::Tag::pt2_compliant_tag});
  m.def("mimo_ss(Tensor A, Tensor B, Tensor C, Tensor? D, Tensor? zi, Tensor x, bool reverse=False) -> (Tensor, Tensor)",
        {at::Tag::pt2_compliant_tag});
  m.def("mimo_ss_grad_sums(Tensor? lam, Tensor? hs, Tensor x, Tensor g, int shared, int want, Tensor? Bm=None, "
        "Tensor? Dm=None) -> Tensor[]",
        {at::Tag::pt2_compliant_tag});
  m.def("lpv_mimo_ss(Tensor A, Tensor B, Tensor C, Tensor? D, Tensor? zi, Tensor x, bool reverse=False, "
        "bool transpose_A=False) -> (Tensor, Tensor)",
        {at::Tag::pt2_compliant_tag});
  m.def("lpv_mimo_ss_states(Tensor A, Tensor B, Tensor C, Tensor? D, Tensor? zi, Tensor x, bool reverse=False, "
        "bool transpose_A=False) -> (Tensor, Tensor, Tensor)",
        {at::Tag::pt2_compliant_tag});
}

TORCH_LIBRARY_IMPL(philtorch, CUDA, m) {
  m.impl("recur2", &recur2_hip);
  m.impl("recurN", &recurN_hip);
  m.impl("lti_recur2", &lti_recur2_hip);
  m.impl("lti_recurN", &lti_recurN_hip);
  m.impl("lti_recur", &lti_recur_hip);
  m.impl("recur", &recur_hip);
  m.impl("recur_backward", &recur_backward_hip);
  m.impl("recurN_backward", &recurN_backward_hip);
  m.impl("lti_recur_backward", &lti_recur_backward_hip);
  m.impl("lti_recurN_backward", &lti_recurN_backward_hip);
  m.impl("sosfilt", &sosfilt_hip);
  m.impl("sosfilt_backward", &sosfilt_backward_hip);
  m.impl("filtfilt", &filtfilt_hip);
  m.impl("filtfilt_backward", &filtfilt_backward_hip);
  m.impl("filtfilt_states", &filtfilt_states_hip);
  m.impl("biquad", &biquad_hip);
  m.impl("biquad_backward", &biquad_backward_hip);
  m.impl("biquad_cols", &biquad_cols_hip);
  m.impl("biquad_cols_backward", &biquad_cols_backward_hip);
  m.impl("lti_ss", &lti_ss_hip);
  m.impl("lfilter_ss", &lfilter_ss_hip);
  m.impl("lti_ss_states", &lti_ss_states_hip);
  m.impl("lfilter_ss_states", &lfilter_ss_states_hip);
  m.impl("lti_ss_backward", &lti_ss_backward_hip);
  m.impl("lfilter_ss_backward", &lfilter_ss_backward_hip);
  m.impl("lpv_ss", &lpv_ss_hip);
  m.impl("lpv_ss_backward", &lpv_ss_backward_hip);
  m.impl("lpv_ss_states", &lpv_ss_states_hip);
  m.impl("mimo_ss", &mimo_ss_hip);
  m.impl("mimo_ss_grad_sums", &mimo_ss_grad_sums_hip);
  m.impl("lpv_mimo_ss", &lpv_mimo_ss_hip);
  m.impl("lpv_mimo_ss_states", &lpv_mimo_ss_states_hip);
}

TORCH_LIBRARY_IMPL(philtorch, CPU, m) {
  m.impl("recur2", &recur2_cpu);
  m.impl("recurN", &recurN_cpu);
  m.impl("lti_recur2", &lti_recur2_cpu);
  m.impl("lti_recurN", &lti_recurN_cpu);
  m.impl("lti_recur", &lti_recur_cpu);
  m.impl("recur", &recur_cpu);
  m.impl("recur_backward", &recur_backward_cpu);
  m.impl("recurN_backward", &recurN_backward_cpu);
  m.impl("lti_recur_backward", &lti_recur_backward_cpu);
  m.impl("lti_recurN_backward", &lti_recurN_backward_cpu);
}
