// C ABI entry points of libphilscan (declared in include/philscan.h) for the
// fixed-order ops: scalar (recur, lti_recur) and 2x2 (recur2, lti_recur2).
// The order-M entry points live in phs_capi_n.hip; both share phs_launch.hpp.
#include "phs_launch.hpp"

namespace phs {
std::atomic<unsigned> g_spin_limit{0};
std::atomic<bool> g_agg_only{false};
std::atomic<int> g_sos_kept_step{-1};
TimingHook g_timing;
TraceHook g_trace;

// ---- workspace of the allocation-free entry point (phs_recur_fwd_noalloc)
// One array per device, held from the library's load until the process
// ends.  Host code never passes `scratch` itself (in host code the name is a
// host-side stand-in, not a device address): it asks each device once for
// the array's address and passes that.
constexpr size_t kScratchBytes = PHS_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

struct ScratchSlot {
  void *ptr = nullptr;  // this device's copy of `scratch`
  uint64_t calls = 0;   // calls since the array was last cleared
};
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
ScratchSlot g_scratch[kMaxDevices];

// Zero-fills n 64-bit words (a kernel, not hipMemsetAsync, so that a
// captured graph replays it as an ordinary node).
__global__ __launch_bounds__(256) void clear_words_kernel(unsigned long long *p, size_t n) {
  for (size_t i = blockIdx.x * size_t(256) + threadIdx.x; i < n; i += size_t(gridDim.x) * 256) p[i] = 0ull;
}
}  // namespace phs

using phs::Block2;
using phs::dispatch;
using phs::Scalar;

extern "C" {

size_t phs_workspace_size(int op, int dtype, int64_t B, int64_t T, int coef_shared, int backward) {
  const bool sh = coef_shared != 0, bw = backward != 0;
  switch (op) {
    case PHS_OP_RECUR: return phs::ws_size<Scalar>(dtype, B, T, true, sh, bw);
    case PHS_OP_LTI_RECUR: return phs::ws_size<Scalar>(dtype, B, T, false, sh, bw);
    case PHS_OP_RECUR2: return phs::ws_size<Block2>(dtype, B, T, true, sh, bw);
    case PHS_OP_LTI_RECUR2: return phs::ws_size<Block2>(dtype, B, T, false, sh, bw);
    default: return 0;
  }
}

const char *phs_error_string(int status) {
  switch (status) {
    case PHS_OK: return "ok";
    case PHS_ERR_INVALID: return "invalid argument (size, null pointer or unsupported combination)";
    case PHS_ERR_WORKSPACE: return "workspace missing or smaller than phs_workspace_size()";
    case PHS_ERR_LAUNCH: return "HIP kernel launch failed";
    case PHS_ERR_DTYPE: return "unsupported dtype";
    case PHS_ERR_TOO_LARGE:
      return "problem needs more workspace than the allocation-free entry point's static scratch "
             "(PHS_NOALLOC_SCRATCH_BYTES); use the entry point that takes a workspace";
    default: return "unknown philscan status";
  }
}

int phs_abi_version(void) { return 112; }

void phs_debug_set_spin_limit(unsigned polls) { phs::g_spin_limit.store(polls, std::memory_order_relaxed); }

void phs_debug_set_aggregates_only(int on) { phs::g_agg_only.store(on != 0, std::memory_order_relaxed); }

void phs_debug_set_sos_kept_step(int step) { phs::g_sos_kept_step.store(step, std::memory_order_relaxed); }

void phs_debug_time_next_launch(void *start_event, void *stop_event) {
  std::lock_guard<std::mutex> lock(phs::g_timing.mu);
  phs::g_timing.start = static_cast<hipEvent_t>(start_event);
  phs::g_timing.stop = static_cast<hipEvent_t>(stop_event);
  phs::g_timing.armed.store(start_event != nullptr || stop_event != nullptr, std::memory_order_release);
}

void phs_debug_trace_next_launch(void *records, size_t n_records) {
  std::lock_guard<std::mutex> lock(phs::g_trace.mu);
  phs::g_trace.records = static_cast<uint64_t *>(records);
  phs::g_trace.n_records = n_records;
  phs::g_trace.armed.store(records != nullptr && n_records > 0, std::memory_order_release);
}

#define PHS_FWD(NAME, ALGT, TV)                                                                    \
  int NAME(int dtype, int64_t B, int64_t T, const void *A, int coef_shared, const void *zi,        \
           const void *x, void *y, void *workspace, size_t workspace_bytes, void *stream) {        \
    return dispatch<ALGT>(dtype, [&](auto alg) {                                                    \
      return phs::launch<decltype(alg)>(B, T, TV, coef_shared != 0, false, A, zi, x, nullptr, y,   \
                                        nullptr, nullptr, workspace, workspace_bytes,              \
                                        static_cast<hipStream_t>(stream));                         \
    });                                                                                            \
  }

#define PHS_BWD(NAME, ALGT, TV)                                                                    \
  int NAME(int dtype, int64_t B, int64_t T, const void *A, int coef_shared, const void *zi,        \
           const void *y, const void *grad_y, void *grad_x, void *grad_A, void *grad_zi,           \
           void *workspace, size_t workspace_bytes, void *stream) {                                \
    return dispatch<ALGT>(dtype, [&](auto alg) {                                                    \
      return phs::launch<decltype(alg)>(B, T, TV, coef_shared != 0, true, A, zi, grad_y, y,        \
                                        grad_x, grad_A, grad_zi, workspace, workspace_bytes,       \
                                        static_cast<hipStream_t>(stream));                         \
    });                                                                                            \
  }

PHS_FWD(phs_recur_fwd, Scalar, true)
PHS_BWD(phs_recur_bwd, Scalar, true)
PHS_FWD(phs_lti_recur_fwd, Scalar, false)
PHS_BWD(phs_lti_recur_bwd, Scalar, false)
PHS_FWD(phs_recur2_fwd, Block2, true)
PHS_BWD(phs_recur2_bwd, Block2, true)
PHS_FWD(phs_lti_recur2_fwd, Block2, false)
PHS_BWD(phs_lti_recur2_bwd, Block2, false)

int phs_recur_fwd_noalloc(int dtype, int64_t B, int64_t T, const void *A, int coef_shared, const void *zi,
                          const void *x, void *y, void *stream) {
  if (B < 0 || T < 0) return PHS_ERR_INVALID;
  if (B == 0 || T == 0) return PHS_OK;
  if (dtype < PHS_F32 || dtype > PHS_I64) return PHS_ERR_DTYPE;
  const size_t need = phs_workspace_size(PHS_OP_RECUR, dtype, B, T, coef_shared, 0);
  if (need == 0) return PHS_ERR_INVALID;
  if (need > phs::kScratchBytes) return PHS_ERR_TOO_LARGE;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= phs::kMaxDevices) return PHS_ERR_LAUNCH;
  hipStream_t s = static_cast<hipStream_t>(stream);
  void *ws = nullptr;
  {
    std::lock_guard<std::mutex> lock(phs::g_scratch_mu);
    phs::ScratchSlot &slot = phs::g_scratch[dev];
    bool clear = false;
    if (!slot.ptr) {
      // set-up on this device's first call, with this device current
      void *p = nullptr;
      if (hipGetSymbolAddress(&p, HIP_SYMBOL(phs::scratch)) != hipSuccess || !p) return PHS_ERR_LAUNCH;
      slot.ptr = p;
      clear = true;
    } else if (++slot.calls >= (uint64_t(1) << 30)) {
      clear = true;  // long before the 32-bit status tags could repeat
    }
    if (clear) {
      slot.calls = 0;
      const size_t words = phs::kScratchBytes / sizeof(unsigned long long);
      hipLaunchKernelGGL(phs::clear_words_kernel, dim3(1024), dim3(256), 0, s,
                         static_cast<unsigned long long *>(slot.ptr), words);
      if (hipGetLastError() != hipSuccess) return PHS_ERR_LAUNCH;
    }
    ws = slot.ptr;
  }
  return phs_recur_fwd(dtype, B, T, A, coef_shared, zi, x, y, ws, phs::kScratchBytes, stream);
}

}  // extern "C"

