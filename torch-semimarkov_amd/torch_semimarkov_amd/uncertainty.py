"""Uncertainty consumers of the streaming backward (reference ``uncertainty.py``).

The reference's streaming uncertainty methods (``uncertainty.py:92-160``,
``:263-328``, ``:330-368``, ``:418-497``) differentiate the log partition with
the CPU PyTorch backward (``use_triton=False``).  Here the same quantities come
from the HIP kernels: the scan backward (``tsm_backward``) gives
d log Z / d cum_scores, and the emission prologue's backward
(``tsm_cum_scores_backward``) carries it to the projected scores.

* :meth:`UncertaintyMixin.compute_boundary_marginals` (streaming):
  ``|d log Z / d cum[:, 1:]|`` summed over labels, optionally divided by its
  per-sequence maximum (``+1e-8``).
* :meth:`UncertaintyMixin.compute_position_marginals`: softmax over labels of
  ``|d log Z / d scores|``.
* :meth:`UncertaintyMixin.compute_entropy_streaming`: entropy of the boundary
  signal normalised to a distribution.
* :meth:`UncertaintyMixin.compute_loss_uncertainty_weighted`:
  ``(1 + lambda * u) * NLL`` with ``u`` from either of the above.

The reference's exact variants (``use_streaming=False``,
``compute_entropy_exact``) materialise the ``(B, T, K, C, C)`` edge tensor for
its non-streaming ``SemiMarkov`` library, which this package does not provide;
they raise ``NotImplementedError``.
"""

from __future__ import annotations

import torch
from torch import Tensor

from .nn import SemiMarkovCRFHead
from .streaming.autograd import semi_crf_streaming_forward
from .streaming.prologue import emission_cum_scores


class UncertaintyMixin:
    """Uncertainty methods for a head with ``projection``, ``transition``,
    ``duration_bias``, ``num_classes`` and ``max_duration`` (reference
    ``uncertainty.py:36-497``)."""

    def _scores(self, hidden_states: Tensor) -> Tensor:
        if self.projection is not None:
            with torch.no_grad():
                return self.projection(hidden_states)
        return hidden_states

    def compute_boundary_marginals(
        self, hidden_states: Tensor, lengths: Tensor, use_streaming: bool = True, normalize: bool = True
    ) -> Tensor:
        """Boundary signal ``(B, T)`` (reference ``uncertainty.py:56-160``)."""
        if not use_streaming:
            raise NotImplementedError(
                "exact boundary marginals need the (B, T, K, C, C) edge tensor of the non-streaming "
                "SemiMarkov library, which the HIP backend does not provide; use use_streaming=True"
            )
        scores = self._scores(hidden_states)
        with torch.enable_grad():
            cum = emission_cum_scores(scores.detach()).requires_grad_(True)
            partition = semi_crf_streaming_forward(
                cum, self.transition.detach(), self.duration_bias.detach(), lengths, self.max_duration,
                semiring="log",
            )
            (grad,) = torch.autograd.grad(partition.sum(), cum)
        signal = grad[:, 1:].abs().sum(dim=-1)
        if normalize:
            signal = signal / (signal.max(dim=-1, keepdim=True)[0] + 1e-8)
        return signal

    def compute_position_marginals(self, hidden_states: Tensor, lengths: Tensor) -> Tensor:
        """Per-position label distribution ``(B, T, C)`` (reference ``uncertainty.py:263-328``)."""
        scores = self._scores(hidden_states)
        with torch.enable_grad():
            s = scores.detach().requires_grad_(True)
            partition = semi_crf_streaming_forward(
                emission_cum_scores(s), self.transition.detach(), self.duration_bias.detach(), lengths,
                self.max_duration, semiring="log",
            )
            (grad,) = torch.autograd.grad(partition.sum(), s)
        return torch.softmax(grad.abs(), dim=-1)

    def compute_entropy_streaming(self, hidden_states: Tensor, lengths: Tensor) -> Tensor:
        """Entropy ``(B,)`` of the normalised boundary signal (reference ``uncertainty.py:330-368``)."""
        p = self.compute_boundary_marginals(hidden_states, lengths, use_streaming=True, normalize=False)
        p = p / (p.sum(dim=-1, keepdim=True) + 1e-8)
        return -(p * torch.log(p.clamp(min=1e-10))).sum(dim=-1)

    def compute_entropy_exact(self, hidden_states: Tensor, lengths: Tensor) -> Tensor:
        """Not provided (reference ``uncertainty.py:370-416`` uses the edge-tensor EntropySemiring)."""
        raise NotImplementedError(
            "exact entropy needs the (B, T, K, C, C) edge tensor of the non-streaming SemiMarkov library "
            "with EntropySemiring, which the HIP backend does not provide; use compute_entropy_streaming"
        )

    def compute_loss_uncertainty_weighted(
        self,
        hidden_states: Tensor,
        lengths: Tensor,
        labels: Tensor,
        uncertainty_weight: float = 1.0,
        focus_mode: str = "high_uncertainty",
        use_triton: bool = False,
        reduction: str = "mean",
    ) -> Tensor:
        """``(1 + uncertainty_weight * u) * NLL`` (reference ``uncertainty.py:418-497``)."""
        with torch.no_grad():
            if focus_mode == "high_uncertainty":
                u = self.compute_entropy_streaming(hidden_states.detach(), lengths)
                u = u / (u.max() + 1e-8)
            elif focus_mode == "boundary_regions":
                u = self.compute_boundary_marginals(hidden_states.detach(), lengths, use_streaming=True).mean(dim=-1)
            else:
                raise ValueError(f"Unknown focus_mode: {focus_mode}")
        res = self.forward(hidden_states, lengths, use_triton)
        nll = res["partition"] - self._score_gold(res["cum_scores"], labels, lengths)
        weighted = nll * (1.0 + uncertainty_weight * u)
        if reduction == "mean":
            return weighted.mean()
        if reduction == "sum":
            return weighted.sum()
        return weighted


class UncertaintySemiMarkovCRFHead(UncertaintyMixin, SemiMarkovCRFHead):
    """:class:`SemiMarkovCRFHead` with the uncertainty methods (reference
    ``uncertainty.py:500-933``): same parameters, initialisation order, loss,
    decoding and traceback."""


__all__ = ["UncertaintyMixin", "UncertaintySemiMarkovCRFHead"]
