"""Independent pins for the oracle (tests only).

* :func:`enumerate_paths` / :func:`brute_log_partition` -- exhaustive
  enumeration of every segmentation of a tiny sequence.  A segmentation is a
  virtual start label ``c0`` followed by segments ``(k_i, c_i)`` with
  ``sum k_i = L`` and ``k_i`` in the allowed durations; its score is
  ``sum_i seg(s_i, k_i, c_i) + trans[c_{i-1}, c_i]`` with ``c_{-1} = c0``.
  This is what the reference recursion computes with ``alpha[0, :] = 0``
  (``streaming/pytorch_reference.py:197-199``): the first segment sums over a
  virtual predecessor label.  log Z is the log-sum-exp over all paths, the
  Viterbi score the max; gradients come from autograd through the explicit
  sum (exact marginals).
* :func:`hmm_forward_backward` -- K=1 special case as a textbook scaled HMM in
  probability space (matrix-vector products), fp64 numpy.  Gives log Z and the
  posterior edge/state counts without any log-semiring recursion.
* :func:`t1_closed_form` -- the known answer of
  ``tests/test_edge_cases.py:167-193`` generalised: for T=1,
  ``log Z = LSE_c(content_c + db[1,c] + LSE_c' trans[c',c])``.
"""

from __future__ import annotations

import itertools
from typing import Optional

import numpy as np
import torch


def allowed_durations(K: int) -> list:
    """Durations 1..K-1; K=1 means unit segments (``pytorch_reference.py:216``)."""
    return [1] if K == 1 else list(range(1, K))


def _compositions(L: int, parts: list):
    if L == 0:
        yield ()
        return
    for p in parts:
        if p <= L:
            for rest in _compositions(L - p, parts):
                yield (p,) + rest


def enumerate_paths(L: int, K: int, C: int):
    """All (c0, [(start, k, label), ...]) segmentations of ``[0, L)``."""
    paths = []
    for comp in _compositions(L, allowed_durations(K)):
        starts = np.cumsum((0,) + comp[:-1])
        for labels in itertools.product(range(C), repeat=len(comp)):
            for c0 in range(C):
                paths.append((c0, list(zip(starts.tolist(), comp, labels))))
    return paths


def path_scores(
    paths,
    cum_b: torch.Tensor,
    transition: torch.Tensor,
    duration_bias: torch.Tensor,
    proj_start_b: Optional[torch.Tensor] = None,
    proj_end_b: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Differentiable score of each path (one sequence; inputs ``(T+1,C)`` etc.)."""
    K = duration_bias.shape[0]
    out = []
    for c0, segs in paths:
        s_total = cum_b.new_zeros(())
        prev = c0
        for (s, k, c) in segs:
            v = cum_b[s + k, c] - cum_b[s, c] + duration_bias[min(k, K - 1), c]
            if proj_start_b is not None:
                v = v + proj_start_b[s, c]
            if proj_end_b is not None:
                v = v + proj_end_b[s + k - 1, c]
            tr = transition[prev, c] if transition.ndim == 2 else transition[k, prev, c]
            s_total = s_total + v + tr
            prev = c
        out.append(s_total)
    return torch.stack(out)


def brute_log_partition(cum, transition, duration_bias, lengths, K, semiring="log",
                        proj_start=None, proj_end=None):
    """Batch of exhaustive partitions (differentiable)."""
    B, Tp1, C = cum.shape
    res = []
    for b in range(B):
        L = int(lengths[b])
        paths = enumerate_paths(L, K, C)
        sc = path_scores(
            paths, cum[b], transition, duration_bias,
            proj_start[b] if proj_start is not None else None,
            proj_end[b] if proj_end is not None else None,
        )
        res.append(torch.logsumexp(sc, 0) if semiring == "log" else sc.max())
    return torch.stack(res)


def brute_viterbi_path(cum_b, transition, duration_bias, K, L):
    """Best path (label sequence of segments) for one sequence -- for traceback checks.

    Returns ``(score, [(start, end, label), ...], margin)`` where ``margin`` is
    the gap to the best path with a *different* segmentation.
    """
    C = cum_b.shape[1]
    paths = enumerate_paths(L, K, C)
    sc = path_scores(paths, cum_b, transition, duration_bias).detach()
    order = torch.argsort(sc, descending=True)
    best = paths[int(order[0])]
    segs_best = [(s, s + k - 1, c) for (s, k, c) in best[1]]
    margin = float("inf")
    for idx in order[1:]:
        p = paths[int(idx)]
        if [(s, s + k - 1, c) for (s, k, c) in p[1]] != segs_best:
            margin = float(sc[order[0]] - sc[idx])
            break
    return float(sc[order[0]]), segs_best, margin


def hmm_forward_backward(cum_b: np.ndarray, transition: np.ndarray, db0: np.ndarray, L: int):
    """K=1 semi-CRF == HMM with emissions ``cum[t+1]-cum[t] + db[0]``.

    Scaled probability-space forward/backward (fp64).  Returns
    ``(logZ, state_post (L, C), trans_counts (C, C), edge_post (L, C, C))`` where
    ``edge_post[t, c', c]`` is P(label at t-1 = c', label at t = c) with the
    virtual label before position 0 summed uniformly (alpha[0] = 1).
    """
    em = (cum_b[1 : L + 1] - cum_b[:L]) + db0[None, :]  # (L, C)
    A = np.exp(transition)  # (C_src, C_dst)
    E = np.exp(em)
    C = A.shape[0]
    alpha = np.zeros((L + 1, C))
    scale = np.zeros(L + 1)
    alpha[0] = 1.0
    scale[0] = 1.0
    for t in range(1, L + 1):
        v = (alpha[t - 1] @ A) * E[t - 1]
        scale[t] = v.sum()
        alpha[t] = v / scale[t]
    logZ = np.log(scale[1:]).sum() + np.log(alpha[L].sum())
    beta = np.zeros((L + 1, C))
    beta[L] = 1.0 / alpha[L].sum()
    for t in range(L, 0, -1):
        beta[t - 1] = A @ (E[t - 1] * beta[t]) / scale[t]
    edge_post = np.zeros((L, C, C))
    for t in range(1, L + 1):
        edge_post[t - 1] = alpha[t - 1][:, None] * A * (E[t - 1] * beta[t])[None, :] / scale[t]
    state_post = edge_post.sum(1)
    return logZ, state_post, edge_post.sum(0), edge_post


def t1_closed_form(cum_b, transition, duration_bias) -> torch.Tensor:
    """T=1 known answer (``tests/test_edge_cases.py:167-193``)."""
    K = duration_bias.shape[0]
    content = cum_b[1] - cum_b[0]
    first = torch.logsumexp(transition, dim=0)  # LSE over c_src for each c_dst
    return torch.logsumexp(content + duration_bias[min(1, K - 1)] + first, 0)
