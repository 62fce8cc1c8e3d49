"""ctypes binding of libtsm_hip.so (C ABI declared in include/tsm_hip.h).

The library is loaded lazily from ``_lib/libtsm_hip.so`` next to this file.
There is no fallback: if the library is missing or fails to load, every GPU
entry point raises :class:`RuntimeError` naming the build command.
"""

from __future__ import annotations

import ctypes
import os
import threading

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libtsm_hip.so")
_lock = threading.Lock()
_lib = None

TSM_SEMIRING_LOG = 0
TSM_SEMIRING_MAX = 1
TSM_DTYPE_F32 = 0
TSM_DTYPE_BF16 = 1
TSM_DTYPE_F16 = 2
TSM_VITERBI_AUTO = 0
TSM_VITERBI_EXACT = 1
TSM_VITERBI_FACTORISED = 2
TSM_NOALLOC_SCRATCH_BYTES = 64 << 20  # include/tsm_hip.h
_ERRORS = {1: ValueError, 2: NotImplementedError, 3: RuntimeError, 4: RuntimeError}

PLAN_FIELDS = (
    "J", "NT", "RS", "P", "Lc", "W", "global_rings", "scan_lds", "NB", "TB",
    "CB", "NCB", "JM", "NTM", "marg_lds", "Kmax", "n_cu", "R", "KP", "RMAX",
    "fast", "FJ", "FR", "FNT", "fast_lds", "mfast", "MR",
    "dense", "DJ", "DNT", "dtrl", "dense_lds", "DG", "DNTM", "DNB", "DTB", "dmarg_lds",
    "coop", "CG", "CCL", "CR", "CNQ", "coop_lds",
    "mfused", "GNB", "GTB",
    "P2", "Lc2", "FRL2", "fast_lds2", "dualF", "dualB", "dualV", "regsF", "regsB", "regsV",
)

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_sz = ctypes.c_size_t

_SIGNATURES = {
    "tsm_version": ([], _i32),
    "tsm_last_error": ([], ctypes.c_char_p),
    "tsm_plan_info": ([_i64, _i64, _i64, _i64, _i64, _i32, _i32, ctypes.POINTER(_i64), _i32], _i32),
    "tsm_forward_workspace": ([_i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, ctypes.POINTER(_sz)], _i32),
    "tsm_forward": (
        [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _p, _p, _p, _p, _p, _p, _sz, _p], _i32),
    "tsm_forward_noalloc": (
        [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _p, _p, _p, _p, _p, _p], _i32),
    "tsm_backward_workspace": ([_i64, _i64, _i64, _i64, _i64, _i32, _i32, ctypes.POINTER(_sz)], _i32),
    "tsm_backward": (
        [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _p, _p, _p, _p,
         _p, _p, _p, _p, _p, _p, _p, _sz, _p], _i32),
    "tsm_viterbi_workspace": ([_i64, _i64, _i64, _i64, _i64, _i32, ctypes.POINTER(_sz)], _i32),
    "tsm_viterbi": (
        [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _i32, _i32, _p, _p, _p, _sz, _p], _i32),
    "tsm_segment_terms": ([_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p, _p], _i32),
    "tsm_prologue_workspace": ([_i64, _i64, _i64, ctypes.POINTER(_sz)], _i32),
    "tsm_cum_scores": ([_p, _i32, _i64, _i64, _i64, _i32, _p, _p, _sz, _p], _i32),
    "tsm_cum_scores_backward": ([_p, _i64, _i64, _i64, _i32, _p, _p, _sz, _p], _i32),
    "tsm_gold_score_workspace": ([_i64, _i64, _i64, _i64, _i64, ctypes.POINTER(_sz)], _i32),
    "tsm_gold_score": ([_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _sz, _p], _i32),
    "tsm_gold_score_backward": (
        [_p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _sz, _p], _i32),
    "tsm_forward_emissions_workspace": ([_i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, ctypes.POINTER(_sz)], _i32),
    "tsm_forward_emissions": (
        [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _p, _p, _p, _p, _p, _p, _sz, _p], _i32),
    "tsm_backward_emissions_workspace": ([_i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, ctypes.POINTER(_sz)], _i32),
    "tsm_backward_emissions": (
        [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _p, _p, _p, _p,
         _p, _p, _p, _p, _p, _p, _p, _sz, _p], _i32),
    "tsm_viterbi_emissions_workspace": ([_i64, _i64, _i64, _i64, _i64, _i32, _i32, ctypes.POINTER(_sz)], _i32),
    "tsm_viterbi_emissions": (
        [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _i32, _i32, _p, _p, _p, _sz, _p], _i32),
    "tsm_gold_score_emissions": ([_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _sz, _p], _i32),
    "tsm_gold_score_emissions_backward": (
        [_p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _sz, _p], _i32),
    "tsm_checkpoint_plan": ([_i64, _i64, _i64, _i64, _i32, _i32, _sz, ctypes.POINTER(_i64), ctypes.POINTER(_i64),
                             ctypes.POINTER(_sz), ctypes.POINTER(_sz)], _i32),
    "tsm_checkpointed_workspace": ([_i64, _i64, _i64, _i64, _i32, _i32, _i64, ctypes.POINTER(_sz),
                                    ctypes.POINTER(_sz)], _i32),
    "tsm_forward_checkpointed": (
        [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _sz, _p], _i32),
    "tsm_backward_checkpointed": (
        [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p,
         _p, _sz, _p], _i32),
    "tsm_ring_checkpoints": ([_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p], _i32),
    "tsm_timing_enable": ([_i32], _i32),
    "tsm_timing_read": ([ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_i64), _i32], _i32),
    "tsm_timing_kernel_count": ([], _i32),
    "tsm_timing_kernel_name": ([_i32], ctypes.c_char_p),
}

EXPORTED = tuple(_SIGNATURES)


def library_path() -> str:
    return _LIB_PATH


def lib():
    """The loaded library (raises RuntimeError if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(_LIB_PATH):
                raise RuntimeError(
                    f"libtsm_hip.so not found at {_LIB_PATH}; build it with "
                    "`python torch-semimarkov_amd/build.py` (or __graft_entry__.build())"
                )
            handle = ctypes.CDLL(_LIB_PATH)
            for name, (args, res) in _SIGNATURES.items():
                fn = getattr(handle, name)
                fn.argtypes = args
                fn.restype = res
            _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().tsm_last_error().decode(errors="replace")
        raise _ERRORS.get(rc, RuntimeError)(f"{what}: {msg}")


def plan_info(B, T, C, K, has_ps=False, has_pe=False, trans_rows=0) -> dict:
    out = (_i64 * len(PLAN_FIELDS))()
    check(lib().tsm_plan_info(B, T, C, K, int(trans_rows), int(has_ps), int(has_pe), out, len(PLAN_FIELDS)),
          "tsm_plan_info")
    return dict(zip(PLAN_FIELDS, [int(v) for v in out]))


def ptr(t) -> int | None:
    """Device address of a tensor (None for a missing optional tensor)."""
    return None if t is None else t.data_ptr()


def timing_enable(on: bool = True) -> None:
    """Start (clearing the totals) or stop per-kernel event timing in the library."""
    check(lib().tsm_timing_enable(int(on)), "tsm_timing_enable")


def timing_read() -> dict:
    """{kernel name: (total ms, launches)} of the kernels timed since timing_enable(True).
    Waits for the recorded events."""
    L = lib()
    n = L.tsm_timing_kernel_count()
    ms = (ctypes.c_double * n)()
    cnt = (_i64 * n)()
    check(L.tsm_timing_read(ms, cnt, n), "tsm_timing_read")
    return {L.tsm_timing_kernel_name(i).decode(): (float(ms[i]), int(cnt[i])) for i in range(n) if cnt[i] > 0}
