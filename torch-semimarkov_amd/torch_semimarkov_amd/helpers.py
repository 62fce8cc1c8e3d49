"""Output types of the Viterbi traceback and gold-segmentation scoring.

``Segment`` / ``ViterbiResult`` mirror ``helpers.py:10-78`` of the reference;
``score_gold_vectorized`` has the signature and semantics of ``helpers.py:365-544``.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor


@dataclass
class Segment:
    """A labelled segment ``[start, end]`` (inclusive ends) with its score contribution."""

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


def score_gold_vectorized(
    cum_scores: Tensor,
    labels: Tensor,
    lengths: Tensor,
    transition: Tensor,
    duration_bias: Tensor,
    max_duration: int,
) -> Tensor:
    r"""Score of the segmentation implied by per-position ``labels``.

    Segments are maximal runs of equal labels inside ``[0, len)``.  A segment
    ``[s, e]`` with label ``c`` contributes ``cum[e+1, c] - cum[s, c]`` +
    ``duration_bias[clamp(e-s+1, 1, K-1), c]`` + ``transition[c_prev, c]`` (no
    transition for the first segment), as in ``helpers.py:365-544``.  For
    ``T == 1`` the duration row is 1 (``helpers.py:410-419``), clamped to the
    table for ``K == 1``.

    Computed with position masks instead of the reference's per-sequence Python
    loop: no host synchronisation, one pass of gathers on the input's device.
    """
    B, Tp1, C = cum_scores.shape
    T = Tp1 - 1
    dev = cum_scores.device
    dtype = cum_scores.dtype
    if T == 0:
        return torch.zeros(B, device=dev, dtype=dtype)
    lengths = lengths.to(device=dev, dtype=torch.long)
    labels = labels.to(device=dev, dtype=torch.long)
    if T == 1:
        l0 = labels[:, 0]
        content = cum_scores[:, 1, :].gather(1, l0.unsqueeze(1)).squeeze(1)
        content = content - cum_scores[:, 0, :].gather(1, l0.unsqueeze(1)).squeeze(1)
        row = min(1, duration_bias.shape[0] - 1)
        return (content + duration_bias[row, l0]) * (lengths > 0).to(dtype)

    pos = torch.arange(T, device=dev)
    valid = pos.unsqueeze(0) < lengths.unsqueeze(1)  # (B, T)
    prev_lab = torch.cat([labels[:, :1], labels[:, :-1]], dim=1)
    next_lab = torch.cat([labels[:, 1:], labels[:, -1:]], dim=1)
    is_start = valid & ((pos == 0).unsqueeze(0) | (labels != prev_lab))
    is_end = valid & ((pos.unsqueeze(0) == lengths.unsqueeze(1) - 1) | (labels != next_lab))

    # content: sum over segment ends of cum[e+1, l] minus sum over starts of cum[s, l]
    lab3 = labels.unsqueeze(-1)
    cum_end = cum_scores[:, 1:, :].gather(2, lab3).squeeze(-1)  # cum[p+1, label[p]]
    cum_beg = cum_scores[:, :-1, :].gather(2, lab3).squeeze(-1)  # cum[p, label[p]]
    content = (cum_end * is_end.to(dtype)).sum(1) - (cum_beg * is_start.to(dtype)).sum(1)

    # duration of the segment ending at p: p - (index of the latest start <= p) + 1
    start_idx = torch.where(is_start, pos.unsqueeze(0).expand(B, T), torch.zeros_like(labels))
    last_start = torch.cummax(start_idx, dim=1).values
    dur = torch.clamp(pos.unsqueeze(0) - last_start + 1, 1, max_duration - 1)
    dsc = duration_bias[dur, labels]  # (B, T)
    dur_term = (dsc * is_end.to(dtype)).sum(1)

    # transitions into every segment start except the first
    tsc = transition[prev_lab, labels]
    trans_term = (tsc * (is_start & (pos > 0).unsqueeze(0)).to(dtype)).sum(1)
    return content + dur_term + trans_term
