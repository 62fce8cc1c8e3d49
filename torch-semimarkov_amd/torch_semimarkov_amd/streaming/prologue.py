"""Emission prologue: projected scores ``(B, T, C)`` -> cumulative scores ``(B, T+1, C)``.

The head builds its cumulative scores as ``zeros(B, T+1, C)`` with
``cumsum(scores.float(), dim=1)`` in rows ``1..T`` (reference ``nn.py:196-209``);
the streaming API asks callers to zero-centre the projected scores first
(``projected - projected.mean(dim=1, keepdim=True)``, reference
``streaming/autograd.py:300-340``, ``streaming/__init__.py:85-121``).
:func:`emission_cum_scores` does both in one HIP pass (``tsm_cum_scores``):
prefix sums carried in fp64 and rounded once to fp32, fp32 / bf16 / fp16
inputs, differentiable (``tsm_cum_scores_backward``: suffix sums).
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import ops

_NATIVE = (torch.float32, torch.bfloat16, torch.float16)


class EmissionCumScores(torch.autograd.Function):
    @staticmethod
    def forward(ctx, scores: Tensor, centre: bool) -> Tensor:
        ctx.centre = bool(centre)
        ctx.dtype = scores.dtype
        return ops.cum_scores(scores.detach().contiguous(), ctx.centre)

    @staticmethod
    def backward(ctx, grad_cum: Tensor):
        g = ops.cum_scores_backward(grad_cum.detach().to(torch.float32).contiguous(), ctx.centre)
        return g.to(ctx.dtype), None


def emission_cum_scores(scores: Tensor, zero_centre: bool = False) -> Tensor:
    """``(B, T+1, C)`` fp32 cumulative scores of ``scores`` ``(B, T, C)``, row 0 = 0.

    ``zero_centre=True`` subtracts each ``(b, c)`` column's mean over all ``T``
    positions first (the streaming API's recommended preprocessing).
    """
    if not isinstance(scores, Tensor) or scores.dim() != 3:
        raise ValueError("scores must be a (batch, T, C) tensor")
    if not scores.is_cuda:
        raise RuntimeError(
            "torch_semimarkov_amd runs on AMD GPUs only: scores is on "
            f"{scores.device}; move the inputs to a ROCm device (e.g. .to('cuda'))"
        )
    B, T, C = scores.shape
    if T == 0:
        return torch.zeros(B, 1, C, device=scores.device, dtype=torch.float32)
    if scores.dtype not in _NATIVE:
        scores = scores.float()
    return EmissionCumScores.apply(scores, bool(zero_centre))


__all__ = ["EmissionCumScores", "emission_cum_scores"]
