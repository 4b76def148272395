// C ABI entry points of libphilscan for a state order M (declared in
// include/philscan.h): recurN and lti_recurN, M = 1..4.  M = 1 and 2 forward
// to the fixed-order entry points (phs_capi.hip); M = 3 and 4 run the generic
// BlockN algebra through launch_blockn / ws_blockn (phs_blockn.hip).
#include <type_traits>

#include "phs_launch.hpp"

namespace phs {
namespace {

// f(order) for the BlockN orders built into the library.
template <class F>
auto with_blockn_order(int M, F &&f) -> decltype(f(std::integral_constant<int, 3>{})) {
  switch (M) {
    case 3: return f(std::integral_constant<int, 3>{});
    case 4: return f(std::integral_constant<int, 4>{});
    default: return decltype(f(std::integral_constant<int, 3>{}))(0);
  }
}

}  // namespace
}  // namespace phs

extern "C" {

size_t phs_workspace_size_n(int op, int dtype, int M, int64_t B, int64_t T, int coef_shared, int backward) {
  switch (op) {
    case PHS_OP_RECUR:
    case PHS_OP_LTI_RECUR: return M == 1 ? phs_workspace_size(op, dtype, B, T, coef_shared, backward) : 0;
    case PHS_OP_RECUR2:
    case PHS_OP_LTI_RECUR2: return M == 2 ? phs_workspace_size(op, dtype, B, T, coef_shared, backward) : 0;
    case PHS_OP_RECURN:
    case PHS_OP_LTI_RECURN: {
      const bool TV = op == PHS_OP_RECURN;
      if (M == 1) return phs_workspace_size(TV ? PHS_OP_RECUR : PHS_OP_LTI_RECUR, dtype, B, T, coef_shared, backward);
      if (M == 2) return phs_workspace_size(TV ? PHS_OP_RECUR2 : PHS_OP_LTI_RECUR2, dtype, B, T, coef_shared, backward);
      return phs::with_blockn_order(M, [&](auto order) -> size_t {
        return phs::ws_blockn<decltype(order)::value>(dtype, B, T, TV, coef_shared != 0, backward != 0);
      });
    }
    default: return 0;
  }
}

#define PHS_FWD_N(NAME, TV, FWD1, FWD2)                                                            \
  int NAME(int dtype, int M, int64_t B, int64_t T, const void *A, int coef_shared, const void *zi, \
           const void *x, void *y, void *workspace, size_t workspace_bytes, void *stream) {        \
    if (M == 1) return FWD1(dtype, B, T, A, coef_shared, zi, x, y, workspace, workspace_bytes, stream); \
    if (M == 2) return FWD2(dtype, B, T, A, coef_shared, zi, x, y, workspace, workspace_bytes, stream); \
    if (M != 3 && M != 4) return PHS_ERR_INVALID;                                                  \
    return phs::with_blockn_order(M, [&](auto order) {                                             \
      return phs::launch_blockn<decltype(order)::value>(dtype, B, T, TV, coef_shared != 0, false,  \
                                                        A, zi, x, nullptr, y, nullptr, nullptr,    \
                                                        workspace, workspace_bytes,                \
                                                        static_cast<hipStream_t>(stream));         \
    });                                                                                            \
  }

#define PHS_BWD_N(NAME, TV, BWD1, BWD2)                                                            \
  int NAME(int dtype, int M, int64_t B, int64_t T, const void *A, int coef_shared, const void *zi, \
           const void *y, const void *grad_y, void *grad_x, void *grad_A, void *grad_zi,           \
           void *workspace, size_t workspace_bytes, void *stream) {                                \
    if (M == 1)                                                                                    \
      return BWD1(dtype, B, T, A, coef_shared, zi, y, grad_y, grad_x, grad_A, grad_zi, workspace,  \
                  workspace_bytes, stream);                                                        \
    if (M == 2)                                                                                    \
      return BWD2(dtype, B, T, A, coef_shared, zi, y, grad_y, grad_x, grad_A, grad_zi, workspace,  \
                  workspace_bytes, stream);                                                        \
    if (M != 3 && M != 4) return PHS_ERR_INVALID;                                                  \
    return phs::with_blockn_order(M, [&](auto order) {                                             \
      return phs::launch_blockn<decltype(order)::value>(dtype, B, T, TV, coef_shared != 0, true,   \
                                                        A, zi, grad_y, y, grad_x, grad_A, grad_zi, \
                                                        workspace, workspace_bytes,                \
                                                        static_cast<hipStream_t>(stream));         \
    });                                                                                            \
  }

PHS_FWD_N(phs_recurN_fwd, true, phs_recur_fwd, phs_recur2_fwd)
PHS_BWD_N(phs_recurN_bwd, true, phs_recur_bwd, phs_recur2_bwd)
PHS_FWD_N(phs_lti_recurN_fwd, false, phs_lti_recur_fwd, phs_lti_recur2_fwd)
PHS_BWD_N(phs_lti_recurN_bwd, false, phs_lti_recur_bwd, phs_lti_recur2_bwd)

}  // extern "C"
