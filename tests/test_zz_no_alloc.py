"""The allocation-free entry point phs_recur_fwd_noalloc (static per-device
scratch instead of a workspace argument) against phs_recur_fwd, through the
C ABI: bit-identical outputs on two calls in a row, the second smaller (the
scratch keeps the first call's contents), both within the parity bar of the
oracle; and the size limit reported without a launch."""
import ctypes

import numpy as np
import pytest

from tests import _data as D

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream():
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


@pytest.fixture(scope="module")
def lib(hip):
    from tests import capi

    return capi.load(), capi


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=lambda d: np.dtype(d).name)
def test_noalloc_matches_workspace_entry_point(lib, dtype):
    import torch

    import oracle

    L, capi = lib
    dt = capi.DTYPES[np.dtype(dtype)]
    for i, (B, T, shared) in enumerate([(24, 200003, False), (3, 7000, True)]):
        g = D.rng(D.seed_of("noalloc", np.dtype(dtype).str, i))
        A = D.coef(g, (T,) if shared else (B, T), dtype)
        zi, x = D.normal(g, (B,), dtype), D.normal(g, (B, T), dtype)
        tA, tz, tx = (torch.from_numpy(v).cuda() for v in (A, zi, x))
        y_ws, y_na = torch.empty_like(tx), torch.full_like(tx, float("nan"))
        need = L.phs_workspace_size(capi.OPS["recur"], dt, B, T, int(shared), 0)
        ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
        print(f"noalloc call {i}: B={B} T={T} {np.dtype(dtype).name} shared={shared}", flush=True)
        rc = L.phs_recur_fwd(dt, B, T, _p(tA), int(shared), _p(tz), _p(tx), _p(y_ws), _p(ws), need, _stream())
        assert rc == capi.PHS_OK, L.phs_error_string(rc)
        rc = L.phs_recur_fwd_noalloc(dt, B, T, _p(tA), int(shared), _p(tz), _p(tx), _p(y_na), _stream())
        assert rc == capi.PHS_OK, L.phs_error_string(rc)
        torch.cuda.synchronize()
        got, ref = y_na.cpu().numpy(), y_ws.cpu().numpy()
        assert np.array_equal(got.view(np.uint8), ref.view(np.uint8)), f"call {i}: outputs differ"
        D.check(got, oracle.recur(A, zi, x), f"call {i} y")


def test_noalloc_size_limit(lib):
    import torch

    L, capi = lib
    x = torch.zeros(16, device="cuda")
    # 100000 one-step rows need 100000 tiles of status words (4.8 MB > 4 MiB)
    rc = L.phs_recur_fwd_noalloc(0, 100000, 1, _p(x), 0, _p(x), _p(x), _p(x), _stream())
    assert rc == capi.PHS_ERR_TOO_LARGE
    assert b"static scratch" in L.phs_error_string(capi.PHS_ERR_TOO_LARGE)
    assert L.phs_recur_fwd_noalloc(0, 0, 5, None, 0, None, None, None, _stream()) == capi.PHS_OK
    assert L.phs_recur_fwd_noalloc(9, 2, 5, _p(x), 0, _p(x), _p(x), _p(x), _stream()) == capi.PHS_ERR_DTYPE
