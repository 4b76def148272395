// Order-M launches of the generic BlockN algebra (declared in
// phs_launch.hpp).  Compiled once per order, with -DPHS_BLOCKN_ORDER=3 and
// -DPHS_BLOCKN_ORDER=4, so that the two sets of instantiations build in
// parallel.  Every template instantiated here names BlockN<T, M> with its
// order explicitly: a helper named alike in both objects but meaning a
// different order would be merged by the linker.
#include "phs_launch.hpp"

#ifndef PHS_BLOCKN_ORDER
#error "compile once per order with -DPHS_BLOCKN_ORDER=3 or -DPHS_BLOCKN_ORDER=4"
#endif

namespace phs {
namespace {

// f(BlockN<T, M>{}) for the element type T of dtype.
template <int M, class F>
int dispatch_blockn_dtype(int dtype, F &&f) {
  switch (dtype) {
    case PHS_F32: return f(BlockN<float, M>{});
    case PHS_F64: return f(BlockN<double, M>{});
    case PHS_C64: return f(BlockN<c64, M>{});
    case PHS_C128: return f(BlockN<c128, M>{});
    case PHS_I64: return f(BlockN<int64_t, M>{});
    default: return PHS_ERR_DTYPE;
  }
}

}  // namespace

template <>
int launch_blockn<PHS_BLOCKN_ORDER>(int dtype, int64_t B, int64_t T, bool TV, bool shared, bool backward,
                                    const void *coef, const void *zi, const void *x, const void *y, void *out,
                                    void *gcoef, void *gzi, void *workspace, size_t ws_bytes, hipStream_t stream) {
  return dispatch_blockn_dtype<PHS_BLOCKN_ORDER>(dtype, [&](auto alg) {
    return launch<decltype(alg)>(B, T, TV, shared, backward, coef, zi, x, y, out, gcoef, gzi, workspace, ws_bytes,
                                 stream);
  });
}

template <>
size_t ws_blockn<PHS_BLOCKN_ORDER>(int dtype, int64_t B, int64_t T, bool TV, bool shared, bool backward) {
  if (B <= 0 || T <= 0) return 0;
  size_t out = 0;
  dispatch_blockn_dtype<PHS_BLOCKN_ORDER>(dtype, [&](auto alg) {
    out = make_layout<decltype(alg)>(B, T, TV, shared, backward).total;
    return 0;
  });
  return out;
}

}  // namespace phs
