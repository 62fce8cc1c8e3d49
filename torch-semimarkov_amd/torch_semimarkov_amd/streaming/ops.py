"""PyTorch custom ops over the C ABI of libtsm_hip.so (namespace ``tsm_amd``).

Each op allocates its outputs and a scratch workspace through the PyTorch
caching allocator on the input's device, then enqueues the HIP kernels on the
current stream of that device (no host synchronisation).  The ops have fake
(meta) implementations, so shapes propagate under tracing.

The ops take already-validated, contiguous fp32 inputs on one HIP device; the
user-facing checks live in :mod:`torch_semimarkov_amd.streaming.autograd`.
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch
from torch import Tensor

from .. import _native as N


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _workspace(nbytes: int, dev: torch.device) -> Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev)


def _size(query, *args) -> int:
    out = ctypes.c_size_t(0)
    N.check(query(*args, ctypes.byref(out)), query.__name__)
    return int(out.value)


def _trans_rows(transition: Tensor) -> int:
    """0 for a static (C, C) transition, else the number of (C, C) matrices."""
    return int(transition.shape[0]) if transition.dim() == 3 else 0


def _check_cooperative(rec: Tensor, B: int, T: int, C: int, K: int, semiring: int, tr_rows: int, what: str) -> None:
    """The cooperative scans (label sets whose rings need several CUs) bound every
    wait on their partner blocks; a group that gives up marks its sequences with
    recomputed = -1 and NaN results.  For those plans only, read the marks (one
    host synchronisation) and raise instead of returning NaN."""
    if tr_rows != 0 or not N.plan_info(B, T, C, K)["coop"]:
        return
    bad = torch.nonzero(rec < 0).flatten().tolist()
    if bad:
        raise RuntimeError(f"{what}: the cooperative scan gave up waiting for its partner blocks "
                           f"(sequences {bad[:8]}); the results would be NaN")


# --------------------------------------------------------------------------- forward
@torch.library.custom_op("tsm_amd::scan_forward", mutates_args=())
def scan_forward(
    cum: Tensor, transition: Tensor, duration_bias: Tensor, lengths: Tensor, K: int, semiring: int,
    proj_start: Optional[Tensor], proj_end: Optional[Tensor], store: bool,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Partition (B,), log2 partition (B,) fp64, alpha_hat, alpha_level, recomputed-chunk counts."""
    lib = N.lib()
    B, Tp1, C = cum.shape
    T = Tp1 - 1
    dev = cum.device
    part = torch.empty(B, device=dev, dtype=torch.float32)
    z2 = torch.empty(B, device=dev, dtype=torch.float64)
    rec = torch.empty(B, device=dev, dtype=torch.int32)
    if store:
        ah = torch.empty(B, Tp1, C, device=dev, dtype=torch.float32)
        al = torch.empty(B, Tp1, device=dev, dtype=torch.float64)
    else:
        ah = torch.empty(0, device=dev, dtype=torch.float32)
        al = torch.empty(0, device=dev, dtype=torch.float64)
    tr_rows = _trans_rows(transition)
    nbytes = _size(lib.tsm_forward_workspace, B, T, C, K, tr_rows, semiring, proj_start is not None,
                   proj_end is not None)
    ws = _workspace(nbytes, dev)
    with torch.cuda.device(dev):
        rc = lib.tsm_forward(
            N.ptr(cum), N.ptr(transition), N.ptr(duration_bias), N.ptr(lengths),
            N.ptr(proj_start), N.ptr(proj_end), B, T, C, K, tr_rows, semiring,
            N.ptr(part), N.ptr(z2), N.ptr(ah) if store else None, N.ptr(al) if store else None,
            N.ptr(rec), N.ptr(ws), ws.numel(), _stream(dev),
        )
    N.check(rc, "tsm_forward")
    _check_cooperative(rec, B, T, C, K, semiring, tr_rows, "tsm_forward")
    return part, z2, ah, al, rec


@scan_forward.register_fake
def _(cum, transition, duration_bias, lengths, K, semiring, proj_start, proj_end, store):
    B, Tp1, C = cum.shape
    part = cum.new_empty(B)
    z2 = cum.new_empty(B, dtype=torch.float64)
    rec = cum.new_empty(B, dtype=torch.int32)
    if store:
        return part, z2, cum.new_empty(B, Tp1, C), cum.new_empty(B, Tp1, dtype=torch.float64), rec
    return part, z2, cum.new_empty(0), cum.new_empty(0, dtype=torch.float64), rec


# --------------------------------------------------------------------------- backward
@torch.library.custom_op("tsm_amd::scan_backward", mutates_args=())
def scan_backward(
    cum: Tensor, transition: Tensor, duration_bias: Tensor, lengths: Tensor, K: int, semiring: int,
    proj_start: Optional[Tensor], proj_end: Optional[Tensor], alpha_hat: Tensor, alpha_level: Tensor,
    log2_partition: Tensor, grad_output: Tensor,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """grad_cum (B,T+1,C), grad_transition (shaped like ``transition``), grad_duration_bias (K,C),
    grad_proj_start, grad_proj_end ((B,T,C) or empty), recomputed-chunk counts (B,)."""
    lib = N.lib()
    B, Tp1, C = cum.shape
    T = Tp1 - 1
    dev = cum.device
    g_cum = torch.empty(B, Tp1, C, device=dev, dtype=torch.float32)
    g_tr = torch.empty(transition.shape, device=dev, dtype=torch.float32)
    g_db = torch.empty(K, C, device=dev, dtype=torch.float32)
    g_ps = torch.empty(B, T, C, device=dev, dtype=torch.float32) if proj_start is not None else None
    g_pe = torch.empty(B, T, C, device=dev, dtype=torch.float32) if proj_end is not None else None
    rec = torch.empty(B, device=dev, dtype=torch.int32)
    tr_rows = _trans_rows(transition)
    nbytes = _size(lib.tsm_backward_workspace, B, T, C, K, tr_rows, proj_start is not None, proj_end is not None)
    ws = _workspace(nbytes, dev)
    with torch.cuda.device(dev):
        rc = lib.tsm_backward(
            N.ptr(cum), N.ptr(transition), N.ptr(duration_bias), N.ptr(lengths),
            N.ptr(proj_start), N.ptr(proj_end), B, T, C, K, tr_rows, semiring,
            N.ptr(alpha_hat), N.ptr(alpha_level), N.ptr(log2_partition), N.ptr(grad_output),
            N.ptr(g_cum), N.ptr(g_tr), N.ptr(g_db), N.ptr(g_ps), N.ptr(g_pe), N.ptr(rec),
            N.ptr(ws), ws.numel(), _stream(dev),
        )
    N.check(rc, "tsm_backward")
    _check_cooperative(rec, B, T, C, K, semiring, tr_rows, "tsm_backward")
    empty = torch.empty(0, device=dev, dtype=torch.float32)
    return g_cum, g_tr, g_db, g_ps if g_ps is not None else empty, g_pe if g_pe is not None else empty.clone(), rec


@scan_backward.register_fake
def _(cum, transition, duration_bias, lengths, K, semiring, proj_start, proj_end, alpha_hat, alpha_level,
      log2_partition, grad_output):
    B, Tp1, C = cum.shape
    g_ps = cum.new_empty(B, Tp1 - 1, C) if proj_start is not None else cum.new_empty(0)
    g_pe = cum.new_empty(B, Tp1 - 1, C) if proj_end is not None else cum.new_empty(0)
    return (cum.new_empty(B, Tp1, C), transition.new_empty(transition.shape), cum.new_empty(K, C), g_ps, g_pe,
            cum.new_empty(B, dtype=torch.int32))


# --------------------------------------------------------------------------- exact Viterbi
@torch.library.custom_op("tsm_amd::viterbi", mutates_args=())
def viterbi(
    cum: Tensor, transition: Tensor, duration_bias: Tensor, lengths: Tensor, K: int,
    proj_start: Optional[Tensor], proj_end: Optional[Tensor], traceback: bool, algorithm: int = 0,
) -> tuple[Tensor, Tensor, Tensor]:
    """Score (B,) fp32; with ``traceback`` also seg_count (B,) int32 and segments (B,T,4) int32
    (start, end, label, previous label; last segment first).  ``algorithm``: 0 auto, 1 exact
    (the reference's fp32 operation order), 2 factorised (see include/tsm_hip.h)."""
    lib = N.lib()
    B, Tp1, C = cum.shape
    T = Tp1 - 1
    dev = cum.device
    score = torch.empty(B, device=dev, dtype=torch.float32)
    if traceback:
        cnt = torch.empty(B, device=dev, dtype=torch.int32)
        segs = torch.empty(B, T, 4, device=dev, dtype=torch.int32)
    else:
        cnt = torch.empty(0, device=dev, dtype=torch.int32)
        segs = torch.empty(0, device=dev, dtype=torch.int32)
    tr_rows = _trans_rows(transition)
    nbytes = _size(lib.tsm_viterbi_workspace, B, T, C, K, tr_rows, int(traceback))
    ws = _workspace(nbytes, dev)
    with torch.cuda.device(dev):
        rc = lib.tsm_viterbi(
            N.ptr(cum), N.ptr(transition), N.ptr(duration_bias), N.ptr(lengths),
            N.ptr(proj_start), N.ptr(proj_end), B, T, C, K, tr_rows, N.ptr(score), int(traceback), int(algorithm),
            N.ptr(cnt) if traceback else None, N.ptr(segs) if traceback else None,
            N.ptr(ws), ws.numel(), _stream(dev),
        )
    N.check(rc, "tsm_viterbi")
    return score, cnt, segs


@viterbi.register_fake
def _(cum, transition, duration_bias, lengths, K, proj_start, proj_end, traceback, algorithm=0):
    B, Tp1, C = cum.shape
    if traceback:
        return (cum.new_empty(B), cum.new_empty(B, dtype=torch.int32),
                cum.new_empty(B, Tp1 - 1, 4, dtype=torch.int32))
    return cum.new_empty(B), cum.new_empty(0, dtype=torch.int32), cum.new_empty(0, dtype=torch.int32)


def segment_terms(cum: Tensor, transition: Tensor, duration_bias: Tensor, seg_count: Tensor, segments: Tensor,
                  K: int) -> Tensor:
    """Score terms of :func:`viterbi`'s traceback rows (``tsm_segment_terms``): (B, T, 6) fp64
    (start, end, label, content, duration bias, transition) for rows i < seg_count[b]; the
    rows after those are unset.  Static (C, C) transitions."""
    lib = N.lib()
    B, Tp1, C = cum.shape
    T = Tp1 - 1
    if transition.dim() != 2:
        raise ValueError("segment_terms: static (C, C) transitions only")
    out = torch.empty(B, T, 6, device=cum.device, dtype=torch.float64)
    with torch.cuda.device(cum.device):
        rc = lib.tsm_segment_terms(N.ptr(cum), N.ptr(transition), N.ptr(duration_bias), N.ptr(seg_count),
                                   N.ptr(segments), B, T, C, int(K), N.ptr(out), _stream(cum.device))
    N.check(rc, "tsm_segment_terms")
    return out


# --------------------------------------------------------------------------- emission prologue
_DTYPES = {torch.float32: N.TSM_DTYPE_F32, torch.bfloat16: N.TSM_DTYPE_BF16, torch.float16: N.TSM_DTYPE_F16}


@torch.library.custom_op("tsm_amd::cum_scores", mutates_args=())
def cum_scores(scores: Tensor, centre: bool) -> Tensor:
    """(B, T+1, C) fp32 prefix sums of ``scores`` (B, T, C) (fp32 / bf16 / fp16), row 0 = 0."""
    lib = N.lib()
    B, T, C = scores.shape
    dev = scores.device
    out = torch.empty(B, T + 1, C, device=dev, dtype=torch.float32)
    ws = _workspace(_size(lib.tsm_prologue_workspace, B, T, C), dev)
    with torch.cuda.device(dev):
        rc = lib.tsm_cum_scores(N.ptr(scores), _DTYPES[scores.dtype], B, T, C, int(centre), N.ptr(out), N.ptr(ws),
                                ws.numel(), _stream(dev))
    N.check(rc, "tsm_cum_scores")
    return out


@cum_scores.register_fake
def _(scores, centre):
    B, T, C = scores.shape
    return scores.new_empty(B, T + 1, C, dtype=torch.float32)


@torch.library.custom_op("tsm_amd::cum_scores_backward", mutates_args=())
def cum_scores_backward(grad_cum: Tensor, centre: bool) -> Tensor:
    """(B, T, C) fp32 gradient of the scores from the gradient of the cumulative scores."""
    lib = N.lib()
    B, Tp1, C = grad_cum.shape
    dev = grad_cum.device
    out = torch.empty(B, Tp1 - 1, C, device=dev, dtype=torch.float32)
    ws = _workspace(_size(lib.tsm_prologue_workspace, B, Tp1 - 1, C), dev)
    with torch.cuda.device(dev):
        rc = lib.tsm_cum_scores_backward(N.ptr(grad_cum), B, Tp1 - 1, C, int(centre), N.ptr(out), N.ptr(ws),
                                         ws.numel(), _stream(dev))
    N.check(rc, "tsm_cum_scores_backward")
    return out


@cum_scores_backward.register_fake
def _(grad_cum, centre):
    B, Tp1, C = grad_cum.shape
    return grad_cum.new_empty(B, Tp1 - 1, C)


# --------------------------------------------------------------------------- gold-path score
@torch.library.custom_op("tsm_amd::gold_score", mutates_args=())
def gold_score(cum: Tensor, transition: Tensor, duration_bias: Tensor, labels: Tensor, lengths: Tensor,
               K: int) -> Tensor:
    """Score (B,) fp32 of the segmentation implied by ``labels`` (B,T) int64; ``transition`` (C,C)."""
    lib = N.lib()
    B, Tp1, C = cum.shape
    T = Tp1 - 1
    dev = cum.device
    Kdb = duration_bias.shape[0]
    score = torch.empty(B, device=dev, dtype=torch.float32)
    ws = _workspace(_size(lib.tsm_gold_score_workspace, B, T, C, K, Kdb), dev)
    with torch.cuda.device(dev):
        rc = lib.tsm_gold_score(N.ptr(cum), N.ptr(transition), N.ptr(duration_bias), N.ptr(labels), N.ptr(lengths),
                                B, T, C, K, Kdb, N.ptr(score), N.ptr(ws), ws.numel(), _stream(dev))
    N.check(rc, "tsm_gold_score")
    return score


@gold_score.register_fake
def _(cum, transition, duration_bias, labels, lengths, K):
    return cum.new_empty(cum.shape[0])


@torch.library.custom_op("tsm_amd::gold_score_backward", mutates_args=())
def gold_score_backward(labels: Tensor, lengths: Tensor, grad_output: Tensor, T: int, C: int, K: int,
                        Kdb: int) -> tuple[Tensor, Tensor, Tensor]:
    """grad_cum (B,T+1,C) (scaled by grad_output), grad_transition (C,C), grad_duration_bias (Kdb,C)."""
    lib = N.lib()
    B = labels.shape[0]
    dev = labels.device
    g_cum = torch.empty(B, T + 1, C, device=dev, dtype=torch.float32)
    g_tr = torch.empty(C, C, device=dev, dtype=torch.float32)
    g_db = torch.empty(Kdb, C, device=dev, dtype=torch.float32)
    ws = _workspace(_size(lib.tsm_gold_score_workspace, B, T, C, K, Kdb), dev)
    with torch.cuda.device(dev):
        rc = lib.tsm_gold_score_backward(N.ptr(labels), N.ptr(lengths), B, T, C, K, Kdb, N.ptr(grad_output),
                                         N.ptr(g_cum), N.ptr(g_tr), N.ptr(g_db), N.ptr(ws), ws.numel(),
                                         _stream(dev))
    N.check(rc, "tsm_gold_score_backward")
    return g_cum, g_tr, g_db


@gold_score_backward.register_fake
def _(labels, lengths, grad_output, T, C, K, Kdb):
    B = labels.shape[0]
    f = grad_output.new_empty
    return f(B, T + 1, C), f(C, C), f(Kdb, C)


# --------------------------------------------------------------------------- emission input
# The same passes on projected scores (B, T, C) fp32 instead of cumulative scores
# (tsm_*_emissions): the register-resident scans read the scores and carry the
# prefix sums themselves, so no (B, T+1, C) tensor is built (see include/tsm_hip.h).
@torch.library.custom_op("tsm_amd::scan_forward_em", mutates_args=())
def scan_forward_em(
    scores: Tensor, transition: Tensor, duration_bias: Tensor, lengths: Tensor, K: int, semiring: int,
    proj_start: Optional[Tensor], proj_end: Optional[Tensor], store: bool,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """As :func:`scan_forward` on ``scores`` (B, T, C), T >= 1."""
    lib = N.lib()
    B, T, C = scores.shape
    dev = scores.device
    part = torch.empty(B, device=dev, dtype=torch.float32)
    z2 = torch.empty(B, device=dev, dtype=torch.float64)
    rec = torch.empty(B, device=dev, dtype=torch.int32)
    if store:
        ah = torch.empty(B, T + 1, C, device=dev, dtype=torch.float32)
        al = torch.empty(B, T + 1, device=dev, dtype=torch.float64)
    else:
        ah = torch.empty(0, device=dev, dtype=torch.float32)
        al = torch.empty(0, device=dev, dtype=torch.float64)
    tr_rows = _trans_rows(transition)
    nbytes = _size(lib.tsm_forward_emissions_workspace, B, T, C, K, tr_rows, semiring, proj_start is not None,
                   proj_end is not None)
    ws = _workspace(nbytes, dev)
    with torch.cuda.device(dev):
        rc = lib.tsm_forward_emissions(
            N.ptr(scores), N.ptr(transition), N.ptr(duration_bias), N.ptr(lengths),
            N.ptr(proj_start), N.ptr(proj_end), B, T, C, K, tr_rows, semiring,
            N.ptr(part), N.ptr(z2), N.ptr(ah) if store else None, N.ptr(al) if store else None,
            N.ptr(rec), N.ptr(ws), ws.numel(), _stream(dev),
        )
    N.check(rc, "tsm_forward_emissions")
    _check_cooperative(rec, B, T, C, K, semiring, tr_rows, "tsm_forward_emissions")
    return part, z2, ah, al, rec


@scan_forward_em.register_fake
def _(scores, transition, duration_bias, lengths, K, semiring, proj_start, proj_end, store):
    B, T, C = scores.shape
    part = scores.new_empty(B)
    z2 = scores.new_empty(B, dtype=torch.float64)
    rec = scores.new_empty(B, dtype=torch.int32)
    if store:
        return part, z2, scores.new_empty(B, T + 1, C), scores.new_empty(B, T + 1, dtype=torch.float64), rec
    return part, z2, scores.new_empty(0), scores.new_empty(0, dtype=torch.float64), rec


@torch.library.custom_op("tsm_amd::scan_backward_em", mutates_args=())
def scan_backward_em(
    scores: Tensor, transition: Tensor, duration_bias: Tensor, lengths: Tensor, K: int, semiring: int,
    proj_start: Optional[Tensor], proj_end: Optional[Tensor], alpha_hat: Tensor, alpha_level: Tensor,
    log2_partition: Tensor, grad_output: Tensor,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """As :func:`scan_backward`, with grad_scores (B, T, C) in place of grad_cum."""
    lib = N.lib()
    B, T, C = scores.shape
    dev = scores.device
    g_sc = torch.empty(B, T, C, device=dev, dtype=torch.float32)
    g_tr = torch.empty(transition.shape, device=dev, dtype=torch.float32)
    g_db = torch.empty(K, C, device=dev, dtype=torch.float32)
    g_ps = torch.empty(B, T, C, device=dev, dtype=torch.float32) if proj_start is not None else None
    g_pe = torch.empty(B, T, C, device=dev, dtype=torch.float32) if proj_end is not None else None
    rec = torch.empty(B, device=dev, dtype=torch.int32)
    tr_rows = _trans_rows(transition)
    nbytes = _size(lib.tsm_backward_emissions_workspace, B, T, C, K, tr_rows, semiring, proj_start is not None,
                   proj_end is not None)
    ws = _workspace(nbytes, dev)
    with torch.cuda.device(dev):
        rc = lib.tsm_backward_emissions(
            N.ptr(scores), N.ptr(transition), N.ptr(duration_bias), N.ptr(lengths),
            N.ptr(proj_start), N.ptr(proj_end), B, T, C, K, tr_rows, semiring,
            N.ptr(alpha_hat), N.ptr(alpha_level), N.ptr(log2_partition), N.ptr(grad_output),
            N.ptr(g_sc), N.ptr(g_tr), N.ptr(g_db), N.ptr(g_ps), N.ptr(g_pe), N.ptr(rec),
            N.ptr(ws), ws.numel(), _stream(dev),
        )
    N.check(rc, "tsm_backward_emissions")
    _check_cooperative(rec, B, T, C, K, semiring, tr_rows, "tsm_backward_emissions")
    empty = torch.empty(0, device=dev, dtype=torch.float32)
    return g_sc, g_tr, g_db, g_ps if g_ps is not None else empty, g_pe if g_pe is not None else empty.clone(), rec


@scan_backward_em.register_fake
def _(scores, transition, duration_bias, lengths, K, semiring, proj_start, proj_end, alpha_hat, alpha_level,
      log2_partition, grad_output):
    B, T, C = scores.shape
    g_ps = scores.new_empty(B, T, C) if proj_start is not None else scores.new_empty(0)
    g_pe = scores.new_empty(B, T, C) if proj_end is not None else scores.new_empty(0)
    return (scores.new_empty(B, T, C), transition.new_empty(transition.shape), scores.new_empty(K, C), g_ps, g_pe,
            scores.new_empty(B, dtype=torch.int32))


@torch.library.custom_op("tsm_amd::viterbi_em", mutates_args=())
def viterbi_em(
    scores: Tensor, transition: Tensor, duration_bias: Tensor, lengths: Tensor, K: int,
    proj_start: Optional[Tensor], proj_end: Optional[Tensor], traceback: bool, algorithm: int = 0,
) -> tuple[Tensor, Tensor, Tensor]:
    """As :func:`viterbi` on ``scores`` (B, T, C), T >= 1."""
    lib = N.lib()
    B, T, C = scores.shape
    dev = scores.device
    score = torch.empty(B, device=dev, dtype=torch.float32)
    if traceback:
        cnt = torch.empty(B, device=dev, dtype=torch.int32)
        segs = torch.empty(B, T, 4, device=dev, dtype=torch.int32)
    else:
        cnt = torch.empty(0, device=dev, dtype=torch.int32)
        segs = torch.empty(0, device=dev, dtype=torch.int32)
    tr_rows = _trans_rows(transition)
    nbytes = _size(lib.tsm_viterbi_emissions_workspace, B, T, C, K, tr_rows, int(traceback), int(algorithm))
    ws = _workspace(nbytes, dev)
    with torch.cuda.device(dev):
        rc = lib.tsm_viterbi_emissions(
            N.ptr(scores), N.ptr(transition), N.ptr(duration_bias), N.ptr(lengths),
            N.ptr(proj_start), N.ptr(proj_end), B, T, C, K, tr_rows, N.ptr(score), int(traceback), int(algorithm),
            N.ptr(cnt) if traceback else None, N.ptr(segs) if traceback else None,
            N.ptr(ws), ws.numel(), _stream(dev),
        )
    N.check(rc, "tsm_viterbi_emissions")
    return score, cnt, segs


@viterbi_em.register_fake
def _(scores, transition, duration_bias, lengths, K, proj_start, proj_end, traceback, algorithm=0):
    B, T, C = scores.shape
    if traceback:
        return (scores.new_empty(B), scores.new_empty(B, dtype=torch.int32),
                scores.new_empty(B, T, 4, dtype=torch.int32))
    return scores.new_empty(B), scores.new_empty(0, dtype=torch.int32), scores.new_empty(0, dtype=torch.int32)


@torch.library.custom_op("tsm_amd::gold_score_em", mutates_args=())
def gold_score_em(scores: Tensor, transition: Tensor, duration_bias: Tensor, labels: Tensor, lengths: Tensor,
                  K: int) -> Tensor:
    """As :func:`gold_score` on ``scores`` (B, T, C): a segment's content is the sum of its scores."""
    lib = N.lib()
    B, T, C = scores.shape
    dev = scores.device
    Kdb = duration_bias.shape[0]
    score = torch.empty(B, device=dev, dtype=torch.float32)
    ws = _workspace(_size(lib.tsm_gold_score_workspace, B, T, C, K, Kdb), dev)
    with torch.cuda.device(dev):
        rc = lib.tsm_gold_score_emissions(N.ptr(scores), N.ptr(transition), N.ptr(duration_bias), N.ptr(labels),
                                          N.ptr(lengths), B, T, C, K, Kdb, N.ptr(score), N.ptr(ws), ws.numel(),
                                          _stream(dev))
    N.check(rc, "tsm_gold_score_emissions")
    return score


@gold_score_em.register_fake
def _(scores, transition, duration_bias, labels, lengths, K):
    return scores.new_empty(scores.shape[0])


@torch.library.custom_op("tsm_amd::gold_score_em_backward", mutates_args=())
def gold_score_em_backward(labels: Tensor, lengths: Tensor, grad_output: Tensor, T: int, C: int, K: int,
                           Kdb: int) -> tuple[Tensor, Tensor, Tensor]:
    """grad_scores (B,T,C) (scaled by grad_output), grad_transition (C,C), grad_duration_bias (Kdb,C)."""
    lib = N.lib()
    B = labels.shape[0]
    dev = labels.device
    g_sc = torch.empty(B, T, C, device=dev, dtype=torch.float32)
    g_tr = torch.empty(C, C, device=dev, dtype=torch.float32)
    g_db = torch.empty(Kdb, C, device=dev, dtype=torch.float32)
    ws = _workspace(_size(lib.tsm_gold_score_workspace, B, T, C, K, Kdb), dev)
    with torch.cuda.device(dev):
        rc = lib.tsm_gold_score_emissions_backward(N.ptr(labels), N.ptr(lengths), B, T, C, K, Kdb,
                                                   N.ptr(grad_output), N.ptr(g_sc), N.ptr(g_tr), N.ptr(g_db),
                                                   N.ptr(ws), ws.numel(), _stream(dev))
    N.check(rc, "tsm_gold_score_emissions_backward")
    return g_sc, g_tr, g_db


@gold_score_em_backward.register_fake
def _(labels, lengths, grad_output, T, C, K, Kdb):
    B = labels.shape[0]
    f = grad_output.new_empty
    return f(B, T, C), f(C, C), f(Kdb, C)


# --------------------------------------------------------------------------- bounded-memory backward
def checkpoint_plan(B: int, T: int, C: int, K: int, has_ps: bool, has_pe: bool,
                    budget_bytes: int = 0) -> tuple[int, int, int, int]:
    """(window, n_windows, forward workspace bytes, backward workspace bytes) of the
    checkpointed forward / backward (``tsm_checkpoint_plan``); raises
    NotImplementedError for problems without a 16-lane fused plan."""
    lib = N.lib()
    w, nw = ctypes.c_int64(0), ctypes.c_int64(0)
    fw, bw = ctypes.c_size_t(0), ctypes.c_size_t(0)
    N.check(lib.tsm_checkpoint_plan(B, T, C, K, int(has_ps), int(has_pe), int(budget_bytes), ctypes.byref(w),
                                    ctypes.byref(nw), ctypes.byref(fw), ctypes.byref(bw)), "tsm_checkpoint_plan")
    return int(w.value), int(nw.value), int(fw.value), int(bw.value)


def _ck_workspace(B: int, T: int, C: int, K: int, has_ps: bool, has_pe: bool, window: int) -> tuple[int, int]:
    lib = N.lib()
    fw, bw = ctypes.c_size_t(0), ctypes.c_size_t(0)
    N.check(lib.tsm_checkpointed_workspace(B, T, C, K, int(has_ps), int(has_pe), window, ctypes.byref(fw),
                                           ctypes.byref(bw)), "tsm_checkpointed_workspace")
    return int(fw.value), int(bw.value)


@torch.library.custom_op("tsm_amd::scan_forward_ck", mutates_args=())
def scan_forward_ck(
    cum: Tensor, transition: Tensor, duration_bias: Tensor, lengths: Tensor, K: int,
    proj_start: Optional[Tensor], proj_end: Optional[Tensor], window: int, n_windows: int,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Log partition (B,), log2 partition (B,) fp64 and the window checkpoints
    (state (nw,B,Kmax,C), levels (nw,B,Kmax), alpha-hat rows (nw,B,C), their levels (nw,B))."""
    lib = N.lib()
    B, Tp1, C = cum.shape
    T = Tp1 - 1
    dev = cum.device
    Kmax = max(K - 1, 1)
    part = torch.empty(B, device=dev, dtype=torch.float32)
    z2 = torch.empty(B, device=dev, dtype=torch.float64)
    ck_st = torch.empty(n_windows, B, Kmax, C, device=dev, dtype=torch.float32)
    ck_lv = torch.empty(n_windows, B, Kmax, device=dev, dtype=torch.float64)
    ck_ah = torch.empty(n_windows, B, C, device=dev, dtype=torch.float32)
    ck_al = torch.empty(n_windows, B, device=dev, dtype=torch.float64)
    fw, _ = _ck_workspace(B, T, C, K, proj_start is not None, proj_end is not None, window)
    ws = _workspace(fw, dev)
    with torch.cuda.device(dev):
        rc = lib.tsm_forward_checkpointed(
            N.ptr(cum), N.ptr(transition), N.ptr(duration_bias), N.ptr(lengths), N.ptr(proj_start), N.ptr(proj_end),
            B, T, C, K, window, N.ptr(part), N.ptr(z2), N.ptr(ck_st), N.ptr(ck_lv), N.ptr(ck_ah), N.ptr(ck_al),
            N.ptr(ws), ws.numel(), _stream(dev),
        )
    N.check(rc, "tsm_forward_checkpointed")
    return part, z2, ck_st, ck_lv, ck_ah, ck_al


@scan_forward_ck.register_fake
def _(cum, transition, duration_bias, lengths, K, proj_start, proj_end, window, n_windows):
    B, Tp1, C = cum.shape
    Kmax = max(K - 1, 1)
    f = cum.new_empty
    return (f(B), f(B, dtype=torch.float64), f(n_windows, B, Kmax, C), f(n_windows, B, Kmax, dtype=torch.float64),
            f(n_windows, B, C), f(n_windows, B, dtype=torch.float64))


@torch.library.custom_op("tsm_amd::scan_backward_ck", mutates_args=())
def scan_backward_ck(
    cum: Tensor, transition: Tensor, duration_bias: Tensor, lengths: Tensor, K: int,
    proj_start: Optional[Tensor], proj_end: Optional[Tensor], window: int, ck_state: Tensor, ck_level: Tensor,
    ck_alpha: Tensor, ck_alpha_level: Tensor, log2_partition: Tensor, grad_output: Tensor,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """As :func:`scan_backward` (log semiring), recomputing alpha window by window
    from the checkpoints of :func:`scan_forward_ck`."""
    lib = N.lib()
    B, Tp1, C = cum.shape
    T = Tp1 - 1
    dev = cum.device
    g_cum = torch.empty(B, Tp1, C, device=dev, dtype=torch.float32)
    g_tr = torch.empty(C, C, device=dev, dtype=torch.float32)
    g_db = torch.empty(K, C, device=dev, dtype=torch.float32)
    g_ps = torch.empty(B, T, C, device=dev, dtype=torch.float32) if proj_start is not None else None
    g_pe = torch.empty(B, T, C, device=dev, dtype=torch.float32) if proj_end is not None else None
    _, bw = _ck_workspace(B, T, C, K, proj_start is not None, proj_end is not None, window)
    ws = _workspace(bw, dev)
    with torch.cuda.device(dev):
        rc = lib.tsm_backward_checkpointed(
            N.ptr(cum), N.ptr(transition), N.ptr(duration_bias), N.ptr(lengths), N.ptr(proj_start), N.ptr(proj_end),
            B, T, C, K, window, N.ptr(ck_state), N.ptr(ck_level), N.ptr(ck_alpha), N.ptr(ck_alpha_level),
            N.ptr(log2_partition), N.ptr(grad_output), N.ptr(g_cum), N.ptr(g_tr), N.ptr(g_db), N.ptr(g_ps),
            N.ptr(g_pe), N.ptr(ws), ws.numel(), _stream(dev),
        )
    N.check(rc, "tsm_backward_checkpointed")
    empty = torch.empty(0, device=dev, dtype=torch.float32)
    return g_cum, g_tr, g_db, g_ps if g_ps is not None else empty, g_pe if g_pe is not None else empty.clone()


@scan_backward_ck.register_fake
def _(cum, transition, duration_bias, lengths, K, proj_start, proj_end, window, ck_state, ck_level, ck_alpha,
      ck_alpha_level, log2_partition, grad_output):
    B, Tp1, C = cum.shape
    g_ps = cum.new_empty(B, Tp1 - 1, C) if proj_start is not None else cum.new_empty(0)
    g_pe = cum.new_empty(B, Tp1 - 1, C) if proj_end is not None else cum.new_empty(0)
    return cum.new_empty(B, Tp1, C), cum.new_empty(C, C), cum.new_empty(K, C), g_ps, g_pe


# --------------------------------------------------------------------------- checkpoints
@torch.library.custom_op("tsm_amd::ring_checkpoints", mutates_args=())
def ring_checkpoints(alpha_hat: Tensor, alpha_level: Tensor, lengths: Tensor, K: int, interval: int,
                     n_ckpt: int) -> Tensor:
    """Reference-layout ring checkpoints (B, n_ckpt, K, C), raw alpha, natural log units."""
    lib = N.lib()
    B, Tp1, C = alpha_hat.shape
    dev = alpha_hat.device
    out = torch.empty(B, n_ckpt, K, C, device=dev, dtype=torch.float32)
    with torch.cuda.device(dev):
        rc = lib.tsm_ring_checkpoints(N.ptr(alpha_hat), N.ptr(alpha_level), N.ptr(lengths), B, Tp1 - 1, C, K,
                                      interval, n_ckpt, N.ptr(out), _stream(dev))
    N.check(rc, "tsm_ring_checkpoints")
    return out


@ring_checkpoints.register_fake
def _(alpha_hat, alpha_level, lengths, K, interval, n_ckpt):
    B, Tp1, C = alpha_hat.shape
    return alpha_hat.new_empty(B, n_ckpt, K, C)
