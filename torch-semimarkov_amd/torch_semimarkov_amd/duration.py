"""Duration bias parameterisation used by :class:`SemiMarkovCRFHead`.

Only the default fully learned table is provided (``duration.py:54-126`` of the
reference: ``DurationDistribution`` base and ``LearnedDuration`` with
``randn(K, C) * init_std`` initialisation, which fixes the random draw order of
the head's parameters).  The head also accepts any ``nn.Module`` whose
``forward()`` returns a ``(K, C)`` tensor.
"""

from __future__ import annotations

from abc import ABC, abstractmethod

import torch
import torch.nn as nn
from torch import Tensor


class DurationDistribution(nn.Module, ABC):
    """Produces a ``(K, C)`` log-space duration bias."""

    def __init__(self, max_duration: int, num_classes: int):
        super().__init__()
        self.max_duration = max_duration
        self.num_classes = num_classes

    @abstractmethod
    def forward(self) -> Tensor:  # pragma: no cover - interface
        raise NotImplementedError


class LearnedDuration(DurationDistribution):
    """Independent learned bias per (duration, class), initialised ``N(0, init_std^2)``."""

    def __init__(self, max_duration: int, num_classes: int, init_std: float = 0.1):
        super().__init__(max_duration, num_classes)
        self.duration_bias = nn.Parameter(torch.randn(max_duration, num_classes) * init_std)

    def forward(self) -> Tensor:
        return self.duration_bias
