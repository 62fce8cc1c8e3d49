"""The allocation-free forward entry point ``tsm_forward_noalloc`` (static
device scratch, no workspace argument) against ``tsm_forward`` with a
caller-provided workspace, both called directly through the C ABI.

The same kernels run on the same plan, so the outputs must be bit-identical.
Two calls in a row on one GPU share the static scratch: the second, on a
smaller problem, must not see anything of the first.
"""

import ctypes

import numpy as np
import pytest
import torch

from conftest import gpu_available

pytestmark = pytest.mark.gpu

from torch_semimarkov_amd import _native as N  # noqa: E402

DEV = torch.device("cuda", 0) if gpu_available() else None


def _problem(B, T, C, K, seed):
    g = torch.Generator().manual_seed(seed)
    em = torch.randn(B, T, C, generator=g)
    cum = torch.zeros(B, T + 1, C)
    cum[:, 1:] = em.cumsum(1)
    tr = 0.1 * torch.randn(C, C, generator=g)
    db = 0.1 * torch.randn(K, C, generator=g)
    L = torch.randint(max(1, T // 2), T + 1, (B,), generator=g)
    L[0] = T
    return [x.to(DEV) for x in (cum, tr, db, L)]


def _outputs(B, T, C, store):
    part = torch.full((B,), float("nan"), device=DEV)
    z2 = torch.full((B,), float("nan"), device=DEV, dtype=torch.float64)
    ah = torch.full((B, T + 1, C), float("nan"), device=DEV) if store else None
    al = torch.full((B, T + 1), float("nan"), device=DEV, dtype=torch.float64) if store else None
    rec = torch.full((B,), -7, device=DEV, dtype=torch.int32)
    return part, z2, ah, al, rec


def _call(noalloc, cum, tr, db, L, K, semiring, store):
    lib = N.lib()
    B, Tp1, C = cum.shape
    T = Tp1 - 1
    part, z2, ah, al, rec = _outputs(B, T, C, store)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    common = (N.ptr(cum), N.ptr(tr), N.ptr(db), N.ptr(L), None, None, B, T, C, K, 0, semiring,
              N.ptr(part), N.ptr(z2), N.ptr(ah), N.ptr(al), N.ptr(rec))
    if noalloc:
        rc = lib.tsm_forward_noalloc(*common, stream)
        N.check(rc, "tsm_forward_noalloc")
    else:
        sz = ctypes.c_size_t(0)
        N.check(lib.tsm_forward_workspace(B, T, C, K, 0, semiring, 0, 0, ctypes.byref(sz)), "tsm_forward_workspace")
        assert sz.value <= N.TSM_NOALLOC_SCRATCH_BYTES, sz.value
        ws = torch.empty(max(1, sz.value), dtype=torch.uint8, device=DEV)
        N.check(lib.tsm_forward(*common, N.ptr(ws), sz.value, stream), "tsm_forward")
    torch.cuda.synchronize()
    return [x.cpu() if x is not None else None for x in (part, z2, ah, al, rec)]


def _same(a, b):
    for x, y in zip(a, b):
        if x is None:
            assert y is None
            continue
        assert torch.equal(x, y) or (x.dtype.is_floating_point and torch.equal(torch.nan_to_num(x, 7.0),
                                                                               torch.nan_to_num(y, 7.0))), (x, y)


@pytest.mark.parametrize("semiring", [N.TSM_SEMIRING_LOG, N.TSM_SEMIRING_MAX])
def test_noalloc_matches_forward_on_two_calls(semiring):
    """A chunked problem with the alpha tables, then a smaller one without."""
    for (B, T, C, K, store, seed) in [(3, 6000, 24, 300, True, 11), (2, 700, 8, 20, False, 12)]:
        args = _problem(B, T, C, K, seed)
        want = _call(False, *args, K, semiring, store)
        got = _call(True, *args, K, semiring, store)
        _same(got, want)
        assert torch.isfinite(got[0]).all()


def test_noalloc_refuses_oversized_problem():
    """A problem whose workspace exceeds the static scratch is refused on the
    host, before anything is launched (the workspace size is checked first)."""
    lib = N.lib()
    B, T, C, K = 1024, 100_000, 64, 300
    sz = ctypes.c_size_t(0)
    N.check(lib.tsm_forward_workspace(B, T, C, K, 0, 0, 0, 0, ctypes.byref(sz)), "tsm_forward_workspace")
    assert sz.value > N.TSM_NOALLOC_SCRATCH_BYTES, sz.value
    x = torch.zeros(16, device=DEV)
    L = torch.zeros(1, device=DEV, dtype=torch.int64)
    part = torch.zeros(1, device=DEV)
    rc = lib.tsm_forward_noalloc(N.ptr(x), N.ptr(x), N.ptr(x), N.ptr(L), None, None, B, T, C, K, 0, 0,
                                 N.ptr(part), None, None, None, None, None)
    assert rc == 2, rc
    assert "static scratch" in lib.tsm_last_error().decode()
