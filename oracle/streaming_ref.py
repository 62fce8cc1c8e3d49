"""PyTorch-CPU restatement of the reference streaming semi-CRF (oracle; tests only).

Every function cites the reference lines it restates (paths relative to the
reference repository root, ``src/torch_semimarkov/...``).  The code is written
from the reference's *semantics*; the forward gathers all durations of a step
at once (one tensor of shape ``(B, k_eff, C_dst, C_src)``) which holds exactly
the values the reference stacks at ``streaming/pytorch_reference.py:233``, so
its ``logsumexp``/``max`` reductions see identical inputs in fp32.

Conventions (``README.md:96-125``, ``streaming/pytorch_reference.py:86-111``):

* ``cum_scores`` is ``(B, T+1, C)`` with row 0 = 0.
* ``edge[b, s, k, c_dst, c_src] = (cum[s+k,c_dst]-cum[s,c_dst]) + db[min(k,K-1),c_dst]
  (+ proj_start[s,c_dst]) (+ proj_end[s+k-1,c_dst]) + transition[c_src,c_dst]``.
* Durations run ``1..K-1``; K=1 uses duration 1 with ``duration_bias[0]``.
* ``NEG_INF = -1e9`` (``streaming/constants.py:10``).

Pinning: forward/backward/traceback are pinned by ``oracle.brute`` (exhaustive
enumeration for tiny T, C, K; K=1 HMM closed form), by the T=1 known answer of
``tests/test_edge_cases.py:167-193``, by fp64 gradcheck, and by the golden
fixtures produced from the reference itself (``tests/golden``).  See
``tests/test_oracle.py``.
"""

from __future__ import annotations

import math
import warnings
from dataclasses import dataclass
from typing import Optional

import torch

NEG_INF = -1e9  # streaming/constants.py:10


# ---------------------------------------------------------------------------
# small helpers
# ---------------------------------------------------------------------------
def checkpoint_interval(T: int, K: int) -> int:
    """``streaming/pytorch_reference.py:25-45``: S = max(K, floor(sqrt(T*K)))."""
    return max(K, int(math.sqrt(T * K)))


def _reduce(x: torch.Tensor, dim: int, semiring: str) -> torch.Tensor:
    if semiring == "log":
        return torch.logsumexp(x, dim=dim)
    return torch.max(x, dim=dim)[0]


def _transition_block(transition: torch.Tensor, ks: torch.Tensor) -> torch.Tensor:
    """transition[c_src, c_dst] laid out destination-first, per duration.

    Returns ``(1, C_dst, C_src)`` for a static matrix or ``(n_k, C_dst, C_src)``
    for duration-dependent transitions (``pytorch_reference.py:104-111``).
    """
    if transition.ndim == 2:
        return transition.transpose(0, 1).unsqueeze(0)
    return transition[ks].transpose(-1, -2)


def edge_blocks(
    cum: torch.Tensor,
    transition: torch.Tensor,
    duration_bias: torch.Tensor,
    start: torch.Tensor,
    ks: torch.Tensor,
    proj_start: Optional[torch.Tensor] = None,
    proj_end: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Edge potentials for segments ``[start[i], start[i]+ks[i])`` -> ``(B, n, C_dst, C_src)``.

    Element-wise the same arithmetic, in the same order, as
    ``compute_edge_block_streaming`` (``pytorch_reference.py:86-111``):
    ``((content + db) + proj_start) + proj_end`` then ``+ transition``.
    """
    K = duration_bias.shape[0]
    content = cum[:, start + ks, :] - cum[:, start, :]  # (B, n, C)
    dur_idx = torch.clamp(ks, max=K - 1)
    seg = content + duration_bias[dur_idx]
    if proj_start is not None:
        seg = seg + proj_start[:, start, :]
    if proj_end is not None:
        seg = seg + proj_end[:, start + ks - 1, :]
    return seg.unsqueeze(-1) + _transition_block(transition, ks).unsqueeze(0)


# ---------------------------------------------------------------------------
# forward
# ---------------------------------------------------------------------------
def forward(
    cum_scores: torch.Tensor,
    transition: torch.Tensor,
    duration_bias: torch.Tensor,
    lengths: torch.Tensor,
    K: int,
    semiring: str = "log",
    proj_start: Optional[torch.Tensor] = None,
    proj_end: Optional[torch.Tensor] = None,
    checkpoint_interval_: Optional[int] = None,
    return_alpha: bool = False,
):
    """Ring-buffer forward; restates ``pytorch_reference.py:116-273``.

    Returns ``(partition (B,), ring_checkpoints (B, n_ckpt, K, C), S)`` and, when
    ``return_alpha``, also the full ``alpha`` table ``(B, T+1, C)`` (row t holds
    the value the reference writes into the ring at step t; rows beyond a
    sequence's length are left at NEG_INF).
    """
    if semiring not in ("log", "max"):
        raise ValueError(f"semiring must be 'log' or 'max', got {semiring!r}")
    B, Tp1, C = cum_scores.shape
    T = Tp1 - 1
    dtype = cum_scores.dtype

    # zero-centring heuristic warning (pytorch_reference.py:173-182)
    mag = cum_scores[:, -1, :].abs().mean()
    if mag > 1000:
        warnings.warn(
            f"cum_scores endpoint magnitude {mag.item():.0f} suggests non-zero-centered input",
            stacklevel=2,
        )

    S = checkpoint_interval(T, K) if checkpoint_interval_ is None else max(checkpoint_interval_, K)
    n_ckpt = (T + S - 1) // S
    lengths = lengths.to(torch.long)

    ckpts = torch.full((B, n_ckpt, K, C), NEG_INF, dtype=dtype)
    ring = torch.full((B, K, C), NEG_INF, dtype=dtype)
    ring[:, 0, :] = 0.0
    ckpts[:, 0] = ring
    final = torch.full((B, C), NEG_INF, dtype=dtype)
    alpha_tab = None
    if return_alpha:
        alpha_tab = torch.full((B, T + 1, C), NEG_INF, dtype=dtype)
        alpha_tab[:, 0, :] = 0.0

    for t in range(1, T + 1):
        active = (t <= lengths).view(B, 1)
        k_eff = min(K - 1, t)
        ks = torch.arange(1, max(k_eff, 1) + 1)
        starts = t - ks
        alpha_prev = ring[:, starts % K, :]  # (B, n, C_src)
        edge = edge_blocks(cum_scores, transition, duration_bias, starts, ks, proj_start, proj_end)
        # contiguous like the reference's torch.stack (the broadcast alone may
        # inherit transition.T's column-major layout and change reduction order)
        scores = (alpha_prev.unsqueeze(-2) + edge).contiguous()  # (B, n, C_dst, C_src)
        alpha_t = _reduce(_reduce(scores, -1, semiring), 1, semiring)

        slot = t % K
        ring[:, slot, :] = torch.where(active, alpha_t, ring[:, slot, :])
        if alpha_tab is not None:
            alpha_tab[:, t, :] = torch.where(active, alpha_t, alpha_tab[:, t, :])
        if t % S == 0 and t // S < n_ckpt:
            ci = t // S
            ckpts[:, ci] = torch.where(active.view(B, 1, 1), ring, ckpts[:, ci])
        is_final = (t == lengths).view(B, 1)
        if bool(is_final.any()):
            final = torch.where(is_final, alpha_t, final)

    partition = _reduce(final, -1, semiring)
    if return_alpha:
        return partition, ckpts, S, alpha_tab
    return partition, ckpts, S


# ---------------------------------------------------------------------------
# backward
# ---------------------------------------------------------------------------
@dataclass
class BackwardResult:
    grad_cum: torch.Tensor  # (B, T+1, C)
    grad_transition: torch.Tensor  # (B, C, C) or (B, K, C, C)  -- per batch element
    grad_duration_bias: torch.Tensor  # (B, K, C)                -- per batch element
    grad_proj_start: Optional[torch.Tensor]
    grad_proj_end: Optional[torch.Tensor]


def backward(
    cum_scores: torch.Tensor,
    transition: torch.Tensor,
    duration_bias: torch.Tensor,
    lengths: torch.Tensor,
    K: int,
    log_Z: torch.Tensor,
    ring_checkpoints: torch.Tensor,
    S: int,
    semiring: str = "log",
    proj_start: Optional[torch.Tensor] = None,
    proj_end: Optional[torch.Tensor] = None,
) -> BackwardResult:
    """Checkpointed forward-backward; restates ``pytorch_reference.py:276-525``.

    Phase 1 recomputes alpha inside each checkpoint segment from the saved ring
    (``:380-423``), Phase 2 walks t downwards accumulating the marginals
    ``exp(alpha[t,c_src] + edge + beta[t+k,c_dst] - logZ)`` into per-batch
    gradients and updating the beta ring (``:425-523``).  With ``semiring="max"``
    alpha/beta use max and the marginals are the same exponentials ("soft
    max-marginals").  Accumulations into shared rows follow the reference's
    ascending-k order.
    """
    B, Tp1, C = cum_scores.shape
    T = Tp1 - 1
    dtype = cum_scores.dtype
    lengths = lengths.to(torch.long)
    eff = max(S, K)

    g_cum = torch.zeros_like(cum_scores)
    if transition.ndim == 2:
        g_tr = torch.zeros(B, C, C, dtype=dtype)
    else:
        g_tr = torch.zeros(B, K, C, C, dtype=dtype)
    g_db = torch.zeros(B, K, C, dtype=dtype)
    g_ps = torch.zeros_like(proj_start) if proj_start is not None else None
    g_pe = torch.zeros_like(proj_end) if proj_end is not None else None

    alpha_seg = torch.full((B, eff + K, C), NEG_INF, dtype=dtype)
    beta_ring = torch.full((B, K, C), NEG_INF, dtype=dtype)
    for b in range(B):
        beta_ring[b, int(lengths[b]) % K, :] = 0.0

    n_ckpt = ring_checkpoints.shape[1]
    for ci in range(n_ckpt - 1, -1, -1):
        s0 = ci * S
        s1 = min((ci + 1) * S, T)
        alpha_seg.fill_(NEG_INF)
        ring = ring_checkpoints[:, ci].clone()
        alpha_seg[:, 0] = ring[:, s0 % K]

        # Phase 1: recompute alpha for s0+1 .. s1-1 (pytorch_reference.py:387-423)
        for t in range(s0 + 1, s1):
            active = (t < lengths).view(B, 1)
            k_eff = min(K - 1, t)
            ks = torch.arange(1, max(k_eff, 1) + 1)
            starts = t - ks
            scores = (ring[:, starts % K, :].unsqueeze(-2) + edge_blocks(
                cum_scores, transition, duration_bias, starts, ks, proj_start, proj_end
            )).contiguous()
            alpha_t = _reduce(_reduce(scores, -1, semiring), 1, semiring)
            ring[:, t % K] = torch.where(active, alpha_t, ring[:, t % K])
            lt = t - s0
            alpha_seg[:, lt] = torch.where(active, alpha_t, alpha_seg[:, lt])

        # Phase 2: beta + marginals, t descending (pytorch_reference.py:426-523)
        for t in range(s1 - 1, s0 - 1, -1):
            alpha_t = alpha_seg[:, t - s0]
            active = t < lengths
            if not bool(active.any()):
                continue
            max_k = min(K - 1, T - t)
            ks_all = torch.arange(1, max(max_k, 1) + 1)
            ends_all = t + ks_all
            valid_all = (ends_all.view(1, -1) <= lengths.view(B, 1)) & active.view(B, 1)
            keep = valid_all.any(0)
            if not bool(keep.any()):
                continue
            ks = ks_all[keep]
            ends = ends_all[keep]
            valid = valid_all[:, keep]  # (B, n)
            starts = torch.full_like(ks, t)
            edge = edge_blocks(cum_scores, transition, duration_bias, starts, ks, proj_start, proj_end)
            beta_next = beta_ring[:, ends % K, :]  # (B, n, C_dst)
            logm = (
                alpha_t.view(B, 1, 1, C) + edge + beta_next.unsqueeze(-1) - log_Z.view(B, 1, 1, 1)
            )
            marg = torch.where(valid.view(B, -1, 1, 1), torch.exp(logm), torch.zeros_like(logm))
            msum = marg.sum(-1)  # (B, n, C_dst)
            g_cum[:, ends, :] += msum  # distinct rows -> one add each
            for i in range(ks.numel()):
                k = int(ks[i])
                g_cum[:, t, :] -= msum[:, i]
                if transition.ndim == 2:
                    g_tr += marg[:, i].transpose(-1, -2)
                else:
                    g_tr[:, k] += marg[:, i].transpose(-1, -2)
                g_db[:, min(k, K - 1), :] += msum[:, i]
                if g_ps is not None:
                    g_ps[:, t, :] += msum[:, i]
                if g_pe is not None:
                    g_pe[:, t + k - 1, :] += msum[:, i]
            sb = torch.where(
                valid.view(B, -1, 1, 1),
                edge + beta_next.unsqueeze(-1),
                torch.full_like(edge, NEG_INF),
            ).contiguous()
            new_beta = _reduce(_reduce(sb, -2, semiring), 1, semiring)
            slot = t % K
            beta_ring[:, slot] = torch.where(active.view(B, 1), new_beta, beta_ring[:, slot])

    return BackwardResult(g_cum, g_tr, g_db, g_ps, g_pe)


def scale_backward(res: BackwardResult, grad_output: torch.Tensor):
    """``streaming/autograd.py:134-150``: per-batch grads times grad_output[b];
    shared grads reduced as sum_b grad_output[b] * grad[b]."""
    g = grad_output
    B = g.shape[0]
    out_cum = res.grad_cum * g.view(B, 1, 1)
    if res.grad_transition.ndim == 3:
        out_tr = torch.einsum("bij,b->ij", res.grad_transition, g)
    else:
        out_tr = torch.einsum("bkij,b->kij", res.grad_transition, g)
    out_db = torch.einsum("bkc,b->kc", res.grad_duration_bias, g)
    out_ps = res.grad_proj_start * g.view(B, 1, 1) if res.grad_proj_start is not None else None
    out_pe = res.grad_proj_end * g.view(B, 1, 1) if res.grad_proj_end is not None else None
    return out_cum, out_tr, out_db, out_ps, out_pe


class StreamingOracleFunction(torch.autograd.Function):
    """autograd wrapper with the contract of ``SemiCRFStreaming``
    (``streaming/autograd.py:33-161``) -- used for gradcheck of the oracle."""

    @staticmethod
    def forward(ctx, cum, trans, db, lengths, K, semiring, ps, pe):
        part, ck, S = forward(
            cum.detach(), trans.detach(), db.detach(), lengths, K, semiring,
            ps.detach() if ps is not None else None,
            pe.detach() if pe is not None else None,
        )
        ctx.save_for_backward(cum, trans, db, lengths, ck, part, ps, pe)
        ctx.K, ctx.semiring, ctx.S = K, semiring, S
        return part

    @staticmethod
    def backward(ctx, g):
        cum, trans, db, lengths, ck, part, ps, pe = ctx.saved_tensors
        res = backward(cum, trans, db, lengths, ctx.K, part, ck, ctx.S, ctx.semiring, ps, pe)
        gc, gt, gd, gps, gpe = scale_backward(res, g)
        return gc, gt, gd, None, None, None, gps, gpe


def streaming_oracle(cum, trans, db, lengths, K, semiring="log", proj_start=None, proj_end=None):
    return StreamingOracleFunction.apply(cum, trans, db, lengths, K, semiring, proj_start, proj_end)


# ---------------------------------------------------------------------------
# Viterbi traceback (nn.py:444-555) and segment scores
# ---------------------------------------------------------------------------
def viterbi_traceback_single(cum_b: torch.Tensor, transition, duration_bias, K: int, seq_len: int):
    """Restates ``SemiMarkovCRFHead._traceback_single`` (``nn.py:444-531``).

    ``cum_b`` is ``(T+1, C)``.  Returns a list of ``(start, end, label, prev_label)``
    tuples (inclusive ends) plus the table's best final score.  Ties: the
    smallest duration wins (strict ``>`` at ``nn.py:494``), then the first
    source label (``max(dim=-1)``), then the first final label (``argmax``).
    """
    C = cum_b.shape[1]
    cum = cum_b.unsqueeze(0)
    # fp32 inputs reproduce the reference's table; fp64 inputs give the exact optimum
    alpha = torch.full((seq_len + 1, C), NEG_INF, dtype=cum_b.dtype)
    alpha[0] = 0.0
    bp_k = torch.zeros((seq_len + 1, C), dtype=torch.long)
    bp_c = torch.zeros((seq_len + 1, C), dtype=torch.long)
    for t in range(1, seq_len + 1):
        k_eff = min(K - 1, t)
        ks = torch.arange(1, max(k_eff, 1) + 1)
        starts = t - ks
        edge = edge_blocks(cum, transition, duration_bias, starts, ks)[0]  # (n, C_dst, C_src)
        cand = (alpha[starts].unsqueeze(-2) + edge).contiguous()
        best_src, arg_src = cand.max(dim=-1)  # (n, C_dst)
        kbest = best_src.argmax(dim=0)  # first k attaining the max
        val = best_src.gather(0, kbest.view(1, -1)).squeeze(0)
        better = val > alpha[t]
        alpha[t] = torch.where(better, val, alpha[t])
        bp_k[t] = torch.where(better, ks[kbest], bp_k[t])
        bp_c[t] = torch.where(better, arg_src.gather(0, kbest.view(1, -1)).squeeze(0), bp_c[t])
    best_c = int(alpha[seq_len].argmax())
    segs = []
    t, c = seq_len, best_c
    while t > 0:
        k = int(bp_k[t, c])
        cp = int(bp_c[t, c])
        if k == 0:
            break
        segs.append((t - k, t - 1, c, cp))
        t, c = t - k, cp
    segs.reverse()
    return segs, float(alpha[seq_len].max())


def segment_score(cum_b, transition, duration_bias, K, start, end, label, prev_label):
    """``nn.py:533-555`` -- Python-float arithmetic on fp32 tensor items."""
    content = (cum_b[end + 1, label] - cum_b[start, label]).item()
    dur = end - start + 1
    db = duration_bias[min(dur, K - 1), label].item()
    tr = 0.0
    if prev_label is not None:
        tr = transition[prev_label, label].item()
    return content + db + tr


# ---------------------------------------------------------------------------
# gold path score (helpers.py:365-544)
# ---------------------------------------------------------------------------
def score_gold(cum, labels, lengths, transition, duration_bias, K):
    """Score of the segmentation implied by per-position labels.

    Restates ``score_gold_vectorized`` (``helpers.py:365-544``): segments are
    maximal runs of equal labels inside ``[0, len)``; each contributes
    ``cum[end+1,l]-cum[start,l] + db[clamp(dur,1,K-1), l] + trans[prev,l]``
    (no transition for the first segment).  T==1 uses ``db[1]`` (``:410-419``).
    """
    B, Tp1, C = cum.shape
    T = Tp1 - 1
    dtype = cum.dtype
    if T == 0:
        return torch.zeros(B, dtype=dtype)
    if T == 1:
        l0 = labels[:, 0]
        content = cum[:, 1, :].gather(1, l0.view(-1, 1)).squeeze(1)
        content = content - cum[:, 0, :].gather(1, l0.view(-1, 1)).squeeze(1)
        return (content + duration_bias[1, l0]) * (lengths > 0).to(dtype)
    out = torch.zeros(B, dtype=dtype)
    for b in range(B):
        L = int(lengths[b])
        if L == 0:
            continue
        lab = labels[b, :L]
        chg = torch.nonzero(lab[:-1] != lab[1:]).flatten()
        starts = torch.cat([torch.zeros(1, dtype=torch.long), chg + 1])
        ends = torch.cat([chg, torch.tensor([L - 1])])
        segl = lab[starts]
        content = cum[b, ends + 1, segl] - cum[b, starts, segl]
        dur = torch.clamp(ends - starts + 1, 1, K - 1)
        dsc = duration_bias[dur, segl]
        prev = torch.cat([torch.zeros(1, dtype=torch.long), segl[:-1]])
        tsc = transition[prev, segl]
        tsc = torch.cat([torch.zeros(1, dtype=dtype), tsc[1:]])
        out[b] = (content + dsc + tsc).sum()
    return out
