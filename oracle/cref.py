"""ctypes wrapper of ``oracle/lib/libsmref.so`` (the C restatement in
``oracle/semimarkov_ref.c``) -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, the fixture generator ``tests/golden/make_config_fixtures.py``
and ``bench.py``'s ``cpu_baseline`` leg use it.  The product package never
imports it.

* :func:`forward` -- fp64 log partition (or max-semiring score) per sequence,
  the reference's ``semi_crf_streaming_forward_pytorch``
  (``streaming/pytorch_reference.py:116-273``) computed in the label-factorised
  form, optionally with the alpha table.
* :func:`backward` -- fp64 per-sequence gradients of the log partition, as the
  reference's ``semi_crf_streaming_backward_pytorch``
  (``streaming/pytorch_reference.py:276-525``) returns them before the
  ``grad_output`` reduction of ``streaming/autograd.py:134-150``.
* :func:`viterbi` -- the direct max recursion with backtrace
  (``nn.py:444-531``): ``dtype=np.float32`` reproduces the reference's fp32
  table bit for bit; ``np.float64`` also reports, per sequence, the smallest
  best-minus-runner-up gap over the decisions the backtrace takes.

Pinning: ``tests/test_oracle.py`` checks every function against
``oracle/streaming_ref.py`` (itself pinned by enumeration, the HMM closed form
and the reference's golden vectors) on random problems, and the backward
against the gradient identities.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libsmref.so")

_lib = None

_dp = ctypes.POINTER(ctypes.c_double)
_fp = ctypes.POINTER(ctypes.c_float)
_i64p = ctypes.POINTER(ctypes.c_int64)
_i32p = ctypes.POINTER(ctypes.c_int32)


def build():
    """Compile the C restatement (``make -C oracle``)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    """Load (building first when absent) ``libsmref.so``."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.smref_forward.argtypes = [_dp, _dp, _dp, _i64p, _dp, _dp] + [ctypes.c_int] * 6 + [_dp, _dp]
        L.smref_forward.restype = ctypes.c_int
        L.smref_backward.argtypes = [_dp, _dp, _dp, _i64p, _dp, _dp] + [ctypes.c_int] * 5 + [_dp] * 6
        L.smref_backward.restype = ctypes.c_int
        for name, rp in (("smref_viterbi_f32", _fp), ("smref_viterbi_f64", _dp)):
            f = getattr(L, name)
            f.argtypes = [rp, rp, rp, _i64p] + [ctypes.c_int] * 5 + [ctypes.c_double, _dp, _i32p, _i32p, _dp, _i32p,
                                                                        _i32p]
            f.restype = ctypes.c_int
        _lib = L
    return _lib


def _np(x, dtype):
    if x is None:
        return None
    if hasattr(x, "detach"):
        x = x.detach().cpu().numpy()
    return np.ascontiguousarray(np.asarray(x, dtype=dtype))


def _ptr(a, p):
    return None if a is None else a.ctypes.data_as(p)


def _threads(n):
    if n:
        return int(n)
    return max(1, min(os.cpu_count() or 1, 16))


def forward(cum, transition, duration_bias, lengths, K, semiring="log", proj_start=None, proj_end=None,
            return_alpha=False, threads=None):
    """fp64 partition ``(B,)`` (and alpha ``(B, T+1, C)`` when asked)."""
    if semiring not in ("log", "max"):
        raise ValueError(f"semiring must be 'log' or 'max', got {semiring!r}")
    cum = _np(cum, np.float64)
    tr, db = _np(transition, np.float64), _np(duration_bias, np.float64)
    if tr.ndim != 2:
        raise ValueError("the C restatement takes a static (C, C) transition")
    ln = _np(lengths, np.int64)
    ps, pe = _np(proj_start, np.float64), _np(proj_end, np.float64)
    B, Tp1, C = cum.shape
    z = np.zeros(B)
    alpha = np.zeros((B, Tp1, C)) if return_alpha else None
    rc = lib().smref_forward(_ptr(cum, _dp), _ptr(tr, _dp), _ptr(db, _dp), _ptr(ln, _i64p), _ptr(ps, _dp),
                             _ptr(pe, _dp), B, Tp1 - 1, C, int(K), 0 if semiring == "log" else 1,
                             _threads(threads), _ptr(z, _dp), _ptr(alpha, _dp))
    if rc:
        raise RuntimeError(f"smref_forward failed ({rc})")
    return (z, alpha) if return_alpha else z


def backward(cum, transition, duration_bias, lengths, K, proj_start=None, proj_end=None, threads=None):
    """fp64 per-sequence gradients of log Z: dict with ``logZ (B,)``,
    ``grad_cum (B, T+1, C)``, ``grad_transition (B, C, C)``,
    ``grad_duration_bias (B, K, C)``, ``grad_proj_start`` / ``grad_proj_end``."""
    cum = _np(cum, np.float64)
    tr, db = _np(transition, np.float64), _np(duration_bias, np.float64)
    if tr.ndim != 2:
        raise ValueError("the C restatement takes a static (C, C) transition")
    ln = _np(lengths, np.int64)
    ps, pe = _np(proj_start, np.float64), _np(proj_end, np.float64)
    B, Tp1, C = cum.shape
    T = Tp1 - 1
    K = int(K)
    z = np.zeros(B)
    gc = np.zeros((B, Tp1, C))
    gt = np.zeros((B, C, C))
    gd = np.zeros((B, K, C))
    gps = np.zeros((B, T, C)) if ps is not None else None
    gpe = np.zeros((B, T, C)) if pe is not None else None
    rc = lib().smref_backward(_ptr(cum, _dp), _ptr(tr, _dp), _ptr(db, _dp), _ptr(ln, _i64p), _ptr(ps, _dp),
                              _ptr(pe, _dp), B, T, C, K, _threads(threads), _ptr(z, _dp), _ptr(gc, _dp),
                              _ptr(gt, _dp), _ptr(gd, _dp), _ptr(gps, _dp), _ptr(gpe, _dp))
    if rc:
        raise RuntimeError(f"smref_backward failed ({rc})")
    return {"logZ": z, "grad_cum": gc, "grad_transition": gt, "grad_duration_bias": gd,
            "grad_proj_start": gps, "grad_proj_end": gpe}


def viterbi(cum, transition, duration_bias, lengths, K, dtype=np.float64, close_thr=1e-3, threads=None):
    """Direct max recursion with backtrace.  Returns ``score (B,)`` (fp64 value of
    the table in ``dtype``), ``segments`` (list per sequence of
    ``(start, end, label, prev_label)``, first segment first) and, for fp64,
    over the decisions the backtrace takes: ``min_gap (B,)`` (smallest nonzero
    best-minus-runner-up gap), ``n_close (B,)`` (nonzero gaps < close_thr) and
    ``n_ties (B,)`` (exact ties: with fp32-valued inputs, a run of one label cut
    into segments whose durations can be reordered at no change of score)."""
    dtype = np.dtype(dtype)
    if dtype not in (np.dtype(np.float32), np.dtype(np.float64)):
        raise ValueError("dtype must be float32 or float64")
    rp = _fp if dtype == np.float32 else _dp
    cum = _np(cum, dtype)
    tr, db = _np(transition, dtype), _np(duration_bias, dtype)
    ln = _np(lengths, np.int64)
    B, Tp1, C = cum.shape
    T = Tp1 - 1
    score = np.zeros(B)
    nseg = np.zeros(B, dtype=np.int32)
    segs = np.zeros((B, T, 4), dtype=np.int32)
    gap = np.zeros(B)
    ncl = np.zeros(B, dtype=np.int32)
    nties = np.zeros(B, dtype=np.int32)
    f = lib().smref_viterbi_f32 if dtype == np.float32 else lib().smref_viterbi_f64
    rc = f(_ptr(cum, rp), _ptr(tr, rp), _ptr(db, rp), _ptr(ln, _i64p), B, T, C, int(K), _threads(threads),
           float(close_thr), _ptr(score, _dp), _ptr(nseg, _i32p), _ptr(segs, _i32p), _ptr(gap, _dp),
           _ptr(ncl, _i32p), _ptr(nties, _i32p))
    if rc:
        raise RuntimeError(f"smref_viterbi failed ({rc})")
    out = {"score": score, "segments": [[tuple(int(v) for v in s) for s in segs[b, : nseg[b]]] for b in range(B)]}
    if dtype == np.float64:
        out["min_gap"] = gap
        out["n_close"] = ncl
        out["n_ties"] = nties
    return out
