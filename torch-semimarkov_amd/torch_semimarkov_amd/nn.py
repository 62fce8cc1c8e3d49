"""CRF head module on the HIP streaming scan.

:class:`SemiMarkovCRFHead` has the constructor, parameters, initialisation
order and methods of the reference's ``SemiMarkovCRFHead`` (``nn.py:55-565``):
``forward`` / ``compute_loss`` / ``decode`` / ``decode_with_traceback``.  The
scan always runs on the GPU.  ``compute_loss`` and ``decode`` hand the projected
scores straight to the scan (:func:`semi_crf_emissions_forward`,
:func:`score_gold_emissions`), whose kernels carry the prefix sums themselves:
the ``(B, T+1, C)`` cumulative scores are built only where the reference's API
returns or reads them (``forward``'s ``"cum_scores"``, the segment scores of
``decode_with_traceback``).  ``decode_with_traceback`` runs the Viterbi with an
on-device backtrace instead of the reference's per-sequence Python loop.
"""

from __future__ import annotations

from typing import Optional, Union

import numpy as np
import torch
import torch.nn as nn
from torch import Tensor

from .duration import DurationDistribution, LearnedDuration
from .helpers import Segment, ViterbiResult, score_gold_emissions, score_gold_vectorized
from .streaming import ops
from .streaming.autograd import prepare_inputs, semi_crf_emissions_forward, semi_crf_streaming_forward
from .streaming.prologue import emission_cum_scores


class SemiMarkovCRFHead(nn.Module):
    r"""Semi-Markov CRF head: projection -> fp32 cumulative scores -> streaming scan.

    Args:
        num_classes (int): number of labels C.
        max_duration (int): K; segments have durations 1..K-1 (K=1: unit segments).
        hidden_dim (int, optional): adds ``nn.Linear(hidden_dim, C)`` when given.
        init_scale (float): std of the ``transition`` / duration-bias initialisation.
        duration_distribution: ``None`` / ``"learned"`` (default) or an ``nn.Module``
            whose ``forward()`` returns a ``(K, C)`` tensor.  The reference's other
            named distributions are not provided by this package.

    Parameters are created in the reference's order (``nn.py:146-162``):
    ``transition = randn(C, C) * init_scale``, then ``LearnedDuration``
    (``randn(K, C) * init_scale``), then the projection, so seeded runs draw the
    same values.
    """

    def __init__(
        self,
        num_classes: int,
        max_duration: int,
        hidden_dim: Optional[int] = None,
        init_scale: float = 0.1,
        duration_distribution: Optional[Union[str, DurationDistribution, nn.Module]] = None,
    ):
        super().__init__()
        self.num_classes = num_classes
        self.max_duration = max_duration
        self.transition = nn.Parameter(torch.randn(num_classes, num_classes) * init_scale)
        if duration_distribution is None or duration_distribution == "learned":
            self.duration_dist = LearnedDuration(max_duration, num_classes, init_std=init_scale)
        elif isinstance(duration_distribution, nn.Module):
            self.duration_dist = duration_distribution
        else:
            raise NotImplementedError(
                f"duration_distribution={duration_distribution!r}: only 'learned' or an nn.Module "
                "producing a (K, C) tensor are supported"
            )
        self.projection = nn.Linear(hidden_dim, num_classes) if hidden_dim is not None else None

    @property
    def duration_bias(self) -> Tensor:
        """The ``(K, C)`` duration bias (``self.duration_dist()``)."""
        return self.duration_dist()

    # ------------------------------------------------------------------ helpers
    def _scores(self, hidden_states: Tensor) -> Tensor:
        """Projected scores ``(B, T, C)`` (``nn.py:197-201``)."""
        scores = self.projection(hidden_states) if self.projection is not None else hidden_states
        if scores.shape[-1] != self.num_classes:
            raise ValueError(f"scores have {scores.shape[-1]} labels, the head {self.num_classes}")
        return scores

    def _cum_scores(self, hidden_states: Tensor) -> Tensor:
        """``(B, T+1, C)`` fp32 prefix sums of the projected scores, row 0 = 0 (``nn.py:196-209``),
        built by the HIP emission prologue (fp64 prefix sums rounded once)."""
        return emission_cum_scores(self._scores(hidden_states))

    # ------------------------------------------------------------------ API
    def forward(self, hidden_states: Tensor, lengths: Tensor, use_triton: bool = True) -> dict:
        """``{"partition": (B,), "cum_scores": (B, T+1, C)}`` (``nn.py:173-222``)."""
        cum = self._cum_scores(hidden_states)
        partition = semi_crf_streaming_forward(
            cum, self.transition, self.duration_bias, lengths, self.max_duration,
            semiring="log", use_triton=use_triton,
        )
        return {"partition": partition, "cum_scores": cum}

    def compute_loss(
        self, hidden_states: Tensor, lengths: Tensor, labels: Tensor, use_triton: bool = True,
        reduction: str = "mean",
    ) -> Tensor:
        """Negative log-likelihood ``log Z - score(gold)`` (``nn.py:224-271``).

        The partition and the gold score are computed from the projected scores
        directly (the scan kernels carry the prefix sums), with the values of the
        reference's ``forward`` + ``score_gold_vectorized`` on ``cum_scores``."""
        scores = self._scores(hidden_states)
        partition = semi_crf_emissions_forward(
            scores, self.transition, self.duration_bias, lengths, self.max_duration, semiring="log",
        )
        gold = score_gold_emissions(
            scores=scores, labels=labels, lengths=lengths, transition=self.transition,
            duration_bias=self.duration_bias, max_duration=self.max_duration,
        )
        nll = partition - gold
        if reduction == "mean":
            return nll.mean()
        if reduction == "sum":
            return nll.sum()
        return nll

    def _score_gold(self, cum_scores: Tensor, labels: Tensor, lengths: Tensor) -> Tensor:
        return score_gold_vectorized(
            cum_scores=cum_scores, labels=labels, lengths=lengths, transition=self.transition,
            duration_bias=self.duration_bias, max_duration=self.max_duration,
        )

    def decode(self, hidden_states: Tensor, lengths: Tensor, use_triton: bool = True) -> Tensor:
        """Viterbi score ``(B,)`` (``nn.py:306-358``), from the projected scores directly."""
        return semi_crf_emissions_forward(
            self._scores(hidden_states), self.transition, self.duration_bias, lengths, self.max_duration,
            semiring="max",
        )

    def decode_with_traceback(
        self, hidden_states: Tensor, lengths: Tensor, max_traceback_length: int = 10000
    ) -> ViterbiResult:
        """Best segmentation with its segments (``nn.py:360-442``).

        Sequences longer than ``max_traceback_length`` (or empty) get ``[]``; their
        scores are still computed.  Segment scores are ``content + duration bias +
        transition`` in Python-float arithmetic on the fp32 terms, as ``nn.py:533-555``
        computes them (the transition of the first segment comes from the best
        virtual start label).
        """
        with torch.no_grad():
            cum = self._cum_scores(hidden_states)
            tr = self.transition.detach()
            db = self.duration_bias.detach()
            cum_p, tr_p, db_p, len_p, _, _ = prepare_inputs(cum, tr, db, lengths, self.max_duration)
            score, cnt, segs = ops.viterbi(cum_p, tr_p, db_p, len_p, self.max_duration, None, None, True)
            B = cum.shape[0]
            # every segment row with its fp32 score terms (start, end, label, content, duration
            # bias, transition; one kernel) in one transfer, the counts and lengths in another
            packed = ops.segment_terms(cum_p, tr_p, db_p, cnt, segs, self.max_duration).cpu().numpy()
            meta = torch.stack([cnt.to(len_p.device).long(), len_p.long()]).cpu().tolist()
            counts, lens = meta
            all_segments: list[list[Segment]] = [[] for _ in range(B)]
            for b in range(B):
                n = counts[b]
                if not (0 < lens[b] <= max_traceback_length and n > 0):
                    continue
                r = packed[b, :n][::-1]  # first segment first
                sc = (r[:, 3] + r[:, 4]) + r[:, 5]  # (content + duration) + transition, fp64 of fp32 terms
                ints = r[:, :3].astype(np.int64)
                all_segments[b] = list(map(Segment, ints[:, 0].tolist(), ints[:, 1].tolist(), ints[:, 2].tolist(),
                                           sc.tolist()))
        return ViterbiResult(scores=score, segments=all_segments)

    def extra_repr(self) -> str:
        parts = [f"num_classes={self.num_classes}", f"max_duration={self.max_duration}"]
        if self.projection is not None:
            parts.append(f"hidden_dim={self.projection.in_features}")
        parts.append(f"duration_dist={self.duration_dist.__class__.__name__}")
        return ", ".join(parts)
