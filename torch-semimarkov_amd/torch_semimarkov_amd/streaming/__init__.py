"""Streaming semi-Markov CRF scan on MI355X (HIP kernels in ``libtsm_hip.so``).

Public names follow the reference's ``torch_semimarkov.streaming`` package
(``streaming/__init__.py:136-177``): ``semi_crf_streaming_forward``, the
autograd function, ``compute_edge_block_streaming``,
``_compute_checkpoint_interval`` and ``NEG_INF``.  The launchers are
``launch_streaming_hip_kernel`` / ``launch_streaming_hip_backward`` (the
reference's Triton launchers' contracts); ``HAS_HIP`` reports whether the
native library is built.  ``emission_cum_scores`` builds the cumulative scores
from projected scores on the GPU (optionally zero-centred).
"""

from __future__ import annotations

import os
from typing import Optional

import torch

from .. import _native
from .autograd import (
    SemiCRFEmissionsHIP,
    SemiCRFStreamingCheckpointedHIP,
    SemiCRFStreamingHIP,
    _compute_checkpoint_interval,
    launch_streaming_hip_backward,
    launch_streaming_hip_kernel,
    semi_crf_emissions_forward,
    semi_crf_streaming_forward,
)
from .constants import NEG_INF
from .prologue import emission_cum_scores

HAS_HIP = os.path.exists(_native.library_path())

# Names of the reference's GPU autograd function and launchers
# (streaming/__init__.py:136-177), for code written against them.  HAS_TRITON
# answers the reference's question "is the GPU backend usable", here the HIP one.
SemiCRFStreamingTriton = SemiCRFStreamingHIP
launch_streaming_triton_kernel = launch_streaming_hip_kernel
launch_streaming_triton_backward = launch_streaming_hip_backward
HAS_TRITON = HAS_HIP


def compute_edge_block_streaming(
    cum_scores: torch.Tensor,
    transition: torch.Tensor,
    duration_bias: torch.Tensor,
    t: int,
    k: int,
    proj_start: Optional[torch.Tensor] = None,
    proj_end: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Edge block ``(B, C_dst, C_src)`` for segments starting at ``t`` with duration ``k``.

    Utility with the reference's signature and arithmetic order
    (``pytorch_reference.py:48-113``): ``((content + db[min(k, K-1)]) + proj_start[t])
    + proj_end[t+k-1]`` broadcast plus ``transition.T`` (or ``transition[k].T``).
    Plain tensor ops on whatever device the inputs live on; the scan kernels
    build edges in registers and never call it.
    """
    content = cum_scores[:, t + k, :] - cum_scores[:, t, :]
    Kdb = duration_bias.shape[0]
    seg = content + duration_bias[min(k, Kdb - 1)]
    if proj_start is not None:
        seg = seg + proj_start[:, t, :]
    if proj_end is not None:
        seg = seg + proj_end[:, t + k - 1, :]
    trans_k = transition if transition.ndim == 2 else transition[k]
    return seg.unsqueeze(-1) + trans_k.T.unsqueeze(0)


__all__ = [
    "semi_crf_streaming_forward",
    "semi_crf_emissions_forward",
    "SemiCRFStreamingHIP",
    "SemiCRFStreamingCheckpointedHIP",
    "SemiCRFEmissionsHIP",
    "SemiCRFStreamingTriton",
    "compute_edge_block_streaming",
    "launch_streaming_hip_kernel",
    "launch_streaming_hip_backward",
    "launch_streaming_triton_kernel",
    "launch_streaming_triton_backward",
    "_compute_checkpoint_interval",
    "NEG_INF",
    "HAS_HIP",
    "HAS_TRITON",
]
