"""ctypes binding of libphilscan's C ABI (include/philscan.h), for the tests.

Loads the in-tree library; on a GPU machine torch must be imported first so
that the HIP runtime torch uses is the one the library binds to.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(REPO, "philtorch_amd", "libphilscan.so")
HEADER = os.path.join(REPO, "include", "philscan.h")

PHS_OK, PHS_ERR_INVALID, PHS_ERR_WORKSPACE, PHS_ERR_LAUNCH, PHS_ERR_DTYPE, PHS_ERR_TOO_LARGE = range(6)
PHS_LPV_A_SHARED, PHS_LPV_A_TRANSPOSED = 1, 2
PHS_MIMO_A_SHARED, PHS_MIMO_B_SHARED, PHS_MIMO_C_SHARED, PHS_MIMO_D_SHARED = 1, 2, 4, 8
PHS_MIMO_A_STEPS, PHS_MIMO_A_STEPS_T = 16, 32
# phs_padmode codes (torch.nn.functional.pad modes)
PADMODES = {"constant": 0, "replicate": 1, "reflect": 2, "circular": 3}
OPS = {"recur": 0, "lti_recur": 1, "recur2": 2, "lti_recur2": 3}
OPS_N = {"recurN": 4, "lti_recurN": 5}  # order-M ops (entry points take M after dtype)
DTYPES = {np.dtype(np.float32): 0, np.dtype(np.float64): 1, np.dtype(np.complex64): 2,
          np.dtype(np.complex128): 3, np.dtype(np.int64): 4}

_FWD_ARGS = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
             ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
_BWD_ARGS = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
             ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
             ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]


def declared_symbols() -> list[str]:
    """Function names declared in include/philscan.h."""
    import re

    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(phs_[a-z0-9_]+)\s*\(", text)))


def load() -> ctypes.CDLL:
    lib = ctypes.CDLL(LIB_PATH)
    for op in OPS:
        getattr(lib, f"phs_{op}_fwd").argtypes = _FWD_ARGS
        getattr(lib, f"phs_{op}_fwd").restype = ctypes.c_int
        getattr(lib, f"phs_{op}_bwd").argtypes = _BWD_ARGS
        getattr(lib, f"phs_{op}_bwd").restype = ctypes.c_int
    lib.phs_workspace_size.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                       ctypes.c_int]
    lib.phs_workspace_size.restype = ctypes.c_size_t
    for op in OPS_N:
        getattr(lib, f"phs_{op}_fwd").argtypes = [_FWD_ARGS[0], ctypes.c_int, *_FWD_ARGS[1:]]
        getattr(lib, f"phs_{op}_fwd").restype = ctypes.c_int
        getattr(lib, f"phs_{op}_bwd").argtypes = [_BWD_ARGS[0], ctypes.c_int, *_BWD_ARGS[1:]]
        getattr(lib, f"phs_{op}_bwd").restype = ctypes.c_int
    lib.phs_workspace_size_n.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
                                         ctypes.c_int, ctypes.c_int]
    lib.phs_workspace_size_n.restype = ctypes.c_size_t
    lib.phs_error_string.argtypes = [ctypes.c_int]
    lib.phs_error_string.restype = ctypes.c_char_p
    lib.phs_debug_set_spin_limit.argtypes = [ctypes.c_uint]
    lib.phs_debug_set_spin_limit.restype = None
    lib.phs_debug_set_aggregates_only.argtypes = [ctypes.c_int]
    lib.phs_debug_set_aggregates_only.restype = None
    lib.phs_debug_set_sos_kept_step.argtypes = [ctypes.c_int]
    lib.phs_debug_set_sos_kept_step.restype = None
    lib.phs_debug_time_next_launch.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.phs_debug_time_next_launch.restype = None
    lib.phs_debug_trace_next_launch.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    lib.phs_debug_trace_next_launch.restype = None
    lib.phs_stream_probe.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_void_p,
                                     ctypes.c_void_p, ctypes.c_void_p]
    lib.phs_stream_probe.restype = ctypes.c_int
    lib.phs_recur_fwd_noalloc.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                                          ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.phs_recur_fwd_noalloc.restype = ctypes.c_int
    # fused cascade of second-order sections
    lib.phs_sosfilt_workspace_size.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                               ctypes.c_int]
    lib.phs_sosfilt_workspace_size.restype = ctypes.c_size_t
    lib.phs_sosfilt_ckpt_size.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int]
    lib.phs_sosfilt_ckpt_size.restype = ctypes.c_size_t
    lib.phs_sosfilt_fwd.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p,
                                    ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                    ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                    ctypes.c_void_p]
    lib.phs_sosfilt_fwd.restype = ctypes.c_int
    lib.phs_sosfilt_bwd.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p,
                                    ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                    ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                    ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    lib.phs_sosfilt_bwd.restype = ctypes.c_int
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.phs_biquad_fwd.argtypes = [ctypes.c_int, i64, i64, vp, ctypes.c_int, i64, vp, i64, vp, vp, vp, vp, vp, vp,
                                   ctypes.c_size_t, vp]
    lib.phs_biquad_fwd.restype = ctypes.c_int
    lib.phs_biquad_bwd.argtypes = [ctypes.c_int, i64, i64, vp, ctypes.c_int, i64, vp, i64, vp, vp, vp, vp, vp, vp,
                                   vp, vp, vp, ctypes.c_size_t, vp]
    lib.phs_biquad_bwd.restype = ctypes.c_int
    ci = ctypes.c_int
    lib.phs_biquad_bwd_cols.argtypes = [ci, i64, i64, vp, ci, i64, vp, i64, vp, vp, vp, vp, vp, vp, ci, ci, vp, ci,
                                        ci, vp, vp, ctypes.c_size_t, vp]
    lib.phs_biquad_bwd_cols.restype = ctypes.c_int
    # zero-phase biquad filter
    lib.phs_filtfilt_workspace_size.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64]
    lib.phs_filtfilt_workspace_size.restype = ctypes.c_size_t
    lib.phs_filtfilt_mid_size.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64]
    lib.phs_filtfilt_mid_size.restype = ctypes.c_size_t
    lib.phs_filtfilt_fwd.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                                     ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64,
                                     ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_size_t, ctypes.c_void_p]
    lib.phs_filtfilt_fwd.restype = ctypes.c_int
    lib.phs_filtfilt_bwd_scratch_size.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
                                                  ctypes.c_int64, ctypes.c_int]
    lib.phs_filtfilt_bwd_scratch_size.restype = ctypes.c_size_t
    lib.phs_filtfilt_bwd.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                                     ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64,
                                     ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                     ctypes.c_size_t, ctypes.c_void_p]
    lib.phs_filtfilt_bwd.restype = ctypes.c_int
    # single-input single-output state space and lfilter of order <= 4
    lib.phs_lti_ss_workspace_size.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64]
    lib.phs_lti_ss_workspace_size.restype = ctypes.c_size_t
    lib.phs_lti_ss_fwd.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                                   ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                   ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                   ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                   ctypes.c_void_p]
    lib.phs_lti_ss_fwd.restype = ctypes.c_int
    lib.phs_lfilter_fwd.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                                    ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                    ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                    ctypes.c_size_t, ctypes.c_void_p]
    lib.phs_lfilter_fwd.restype = ctypes.c_int
    lib.phs_lpv_ss_workspace_size.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64]
    lib.phs_lpv_ss_workspace_size.restype = ctypes.c_size_t
    i64, vp = ctypes.c_int64, ctypes.c_void_p
    lib.phs_lpv_ss_fwd.argtypes = [ctypes.c_int, ctypes.c_int, i64, i64, vp, ctypes.c_int, vp, i64, i64, vp, i64, i64,
                                   ctypes.c_int, vp, i64, i64, vp, vp, vp, vp, vp, ctypes.c_size_t, vp]
    lib.phs_lpv_ss_fwd.restype = ctypes.c_int
    lib.phs_lpv_ss_rev.argtypes = lib.phs_lpv_ss_fwd.argtypes
    lib.phs_lpv_ss_rev.restype = ctypes.c_int
    for rev, fwd in (("phs_lti_ss_rev", "phs_lti_ss_fwd"), ("phs_lfilter_rev", "phs_lfilter_fwd")):
        getattr(lib, rev).argtypes = getattr(lib, fwd).argtypes
        getattr(lib, rev).restype = ctypes.c_int
    lib.phs_mimo_ss_workspace_size.argtypes = [ctypes.c_int, ctypes.c_int, i64, i64]
    lib.phs_mimo_ss_workspace_size.restype = ctypes.c_size_t
    ci = ctypes.c_int
    lib.phs_lpv_mimo_ss_workspace_size.argtypes = [ci, ci, i64, i64]
    lib.phs_lpv_mimo_ss_workspace_size.restype = ctypes.c_size_t
    lib.phs_lpv_mimo_ss.argtypes = [ci, ci, ci, ci, i64, i64, vp, ci, vp, vp, vp, ci, vp, vp, vp, vp, ci, vp,
                                    ctypes.c_size_t, vp]
    lib.phs_lpv_mimo_ss.restype = ci
    lib.phs_mimo_ss_grad_sums_scratch_size.argtypes = [ci, i64, i64]
    lib.phs_mimo_ss_grad_sums_scratch_size.restype = ctypes.c_size_t
    lib.phs_mimo_ss_grad_sums.argtypes = [ci, ci, ci, ci, i64, i64, vp, vp, vp, vp, vp, vp, ci, vp, vp, vp, vp, vp,
                                          vp, ctypes.c_size_t, vp]
    lib.phs_mimo_ss_grad_sums.restype = ci
    for name in ("phs_mimo_ss_fwd", "phs_mimo_ss_rev"):
        getattr(lib, name).argtypes = [ci, ci, ci, ci, i64, i64, vp, vp, vp, vp, ci, vp, vp, vp, vp, vp,
                                       ctypes.c_size_t, vp]
        getattr(lib, name).restype = ci
    return lib
