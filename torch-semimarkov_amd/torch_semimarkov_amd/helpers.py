"""Output types of the Viterbi traceback and gold-segmentation scoring.

``Segment`` / ``ViterbiResult`` mirror ``helpers.py:10-78`` of the reference;
``score_gold_vectorized`` has the signature and semantics of ``helpers.py:365-544``
and runs on the GPU (``tsm_gold_score`` of ``libtsm_hip.so``).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor


@dataclass(slots=True)
class Segment:
    """A labelled segment ``[start, end]`` (inclusive ends) with its score contribution.

    The fields of the reference's dataclass (``helpers.py:10-49``); slotted, which
    halves the cost of building the thousands a traceback returns."""

    start: int
    end: int
    label: int
    score: float = 0.0

    @property
    def duration(self) -> int:
        """Number of positions, ``end - start + 1``."""
        return self.end - self.start + 1


@dataclass
class ViterbiResult:
    """Best scores ``(B,)`` and, per sequence, the segments of the best segmentation."""

    scores: Tensor
    segments: list[list[Segment]]


class GoldScoreHIP(torch.autograd.Function):
    """Gold-path score on the GPU (``tsm_gold_score``) with its gradients
    (``tsm_gold_score_backward``) for ``cum_scores``, ``transition`` and ``duration_bias``."""

    @staticmethod
    def forward(ctx, cum, transition, duration_bias, labels, lengths, K):
        from .streaming import ops

        ctx.shape = (cum.shape[1] - 1, cum.shape[2], int(K), duration_bias.shape[0])
        ctx.save_for_backward(labels, lengths)
        return ops.gold_score(cum.detach(), transition.detach(), duration_bias.detach(), labels, lengths, int(K))

    @staticmethod
    def backward(ctx, grad_output):
        from .streaming import ops

        labels, lengths = ctx.saved_tensors
        T, C, K, Kdb = ctx.shape
        g = grad_output.detach().to(torch.float32).contiguous()
        g_cum, g_tr, g_db = ops.gold_score_backward(labels, lengths, g, T, C, K, Kdb)
        return g_cum, g_tr, g_db, None, None, None


class GoldScoreEmissionsHIP(torch.autograd.Function):
    """:class:`GoldScoreHIP` on the projected scores ``(B, T, C)``
    (``tsm_gold_score_emissions`` / ``_backward``): a segment's content is the sum
    of its positions' scores."""

    @staticmethod
    def forward(ctx, scores, transition, duration_bias, labels, lengths, K):
        from .streaming import ops

        ctx.shape = (scores.shape[1], scores.shape[2], int(K), duration_bias.shape[0])
        ctx.save_for_backward(labels, lengths)
        return ops.gold_score_em(scores.detach(), transition.detach(), duration_bias.detach(), labels, lengths,
                                 int(K))

    @staticmethod
    def backward(ctx, grad_output):
        from .streaming import ops

        labels, lengths = ctx.saved_tensors
        T, C, K, Kdb = ctx.shape
        g = grad_output.detach().to(torch.float32).contiguous()
        g_sc, g_tr, g_db = ops.gold_score_em_backward(labels, lengths, g, T, C, K, Kdb)
        return g_sc, g_tr, g_db, None, None, None


def score_gold_vectorized(
    cum_scores: Tensor,
    labels: Tensor,
    lengths: Tensor,
    transition: Tensor,
    duration_bias: Tensor,
    max_duration: int,
) -> Tensor:
    r"""Score of the segmentation implied by per-position ``labels`` ``(B, T)``.

    Signature and semantics of the reference's ``score_gold_vectorized``
    (``helpers.py:365-544``): segments are maximal runs of equal labels inside
    ``[0, len)``; a segment ``[s, e]`` with label ``c`` contributes
    ``cum[e+1, c] - cum[s, c]`` + ``duration_bias[clamp(e-s+1, 1, K-1), c]`` +
    ``transition[c_prev, c]`` (no transition for the first segment).  ``T == 1``
    uses duration row 1 (``helpers.py:410-419``).  A ``(K, C, C)`` transition is
    indexed as the reference's flat ``transition.view(-1)[c_prev * C + c]``, i.e.
    its first matrix.

    Runs the HIP kernels of ``libtsm_hip.so`` (one pass over the labels, no host
    synchronisation, fp64 sums); differentiable in ``cum_scores``,
    ``transition`` and ``duration_bias``.  A sequence holding a label outside
    ``[0, C)`` scores NaN.
    """
    B, Tp1, C = cum_scores.shape
    T = Tp1 - 1
    dev = cum_scores.device
    out_dtype = cum_scores.dtype if cum_scores.is_floating_point() else torch.float32
    if T == 0:
        return torch.zeros(B, device=dev, dtype=out_dtype)
    if not cum_scores.is_cuda:
        raise RuntimeError(
            "torch_semimarkov_amd runs on AMD GPUs only: cum_scores is on "
            f"{cum_scores.device}; move the inputs to a ROCm device (e.g. .to('cuda'))"
        )
    if labels.shape != (B, T):
        raise ValueError(f"labels must be ({B}, {T}), got {tuple(labels.shape)}")
    if lengths.shape != (B,):
        raise ValueError(f"lengths must be ({B},), got {tuple(lengths.shape)}")
    tr = transition[0] if transition.dim() == 3 else transition
    if tr.shape != (C, C):
        raise ValueError(f"transition must be ({C}, {C}) or (K, {C}, {C}), got {tuple(transition.shape)}")
    if duration_bias.dim() != 2 or duration_bias.shape[1] != C:
        raise ValueError(f"duration_bias must be (K, {C}), got {tuple(duration_bias.shape)}")
    f32 = lambda x: (x if x.dtype == torch.float32 else x.float()).contiguous()
    score = GoldScoreHIP.apply(
        f32(cum_scores), f32(tr), f32(duration_bias),
        labels.to(device=dev, dtype=torch.int64).contiguous(),
        lengths.to(device=dev, dtype=torch.int64).contiguous(),
        int(max_duration),
    )
    return score if score.dtype == out_dtype else score.to(out_dtype)


def score_gold_emissions(
    scores: Tensor,
    labels: Tensor,
    lengths: Tensor,
    transition: Tensor,
    duration_bias: Tensor,
    max_duration: int,
) -> Tensor:
    r""":func:`score_gold_vectorized` of ``cum_scores = [0, cumsum(scores, dim=1)]``,
    from the projected scores ``(B, T, C)`` directly (a segment's content is the
    sum of its scores); differentiable in ``scores``, ``transition`` and
    ``duration_bias``.  No reference counterpart (the reference scores the gold
    path from ``cum_scores``, ``helpers.py:365-544``)."""
    B, T, C = scores.shape
    dev = scores.device
    out_dtype = scores.dtype if scores.is_floating_point() else torch.float32
    if T == 0:
        return torch.zeros(B, device=dev, dtype=out_dtype)
    if not scores.is_cuda:
        raise RuntimeError(
            "torch_semimarkov_amd runs on AMD GPUs only: scores is on "
            f"{scores.device}; move the inputs to a ROCm device (e.g. .to('cuda'))"
        )
    if labels.shape != (B, T):
        raise ValueError(f"labels must be ({B}, {T}), got {tuple(labels.shape)}")
    if lengths.shape != (B,):
        raise ValueError(f"lengths must be ({B},), got {tuple(lengths.shape)}")
    tr = transition[0] if transition.dim() == 3 else transition
    if tr.shape != (C, C):
        raise ValueError(f"transition must be ({C}, {C}) or (K, {C}, {C}), got {tuple(transition.shape)}")
    if duration_bias.dim() != 2 or duration_bias.shape[1] != C:
        raise ValueError(f"duration_bias must be (K, {C}), got {tuple(duration_bias.shape)}")
    f32 = lambda x: (x if x.dtype == torch.float32 else x.float()).contiguous()
    score = GoldScoreEmissionsHIP.apply(
        f32(scores), f32(tr), f32(duration_bias),
        labels.to(device=dev, dtype=torch.int64).contiguous(),
        lengths.to(device=dev, dtype=torch.int64).contiguous(),
        int(max_duration),
    )
    return score if score.dtype == out_dtype else score.to(out_dtype)
