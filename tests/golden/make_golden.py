"""Generate golden vectors from the reference implementation (run in the build container only).

Usage (from the repository root, with the reference checked out read-only)::

    PYTHONDONTWRITEBYTECODE=1 python tests/golden/make_golden.py /root/reference/src

The reference is imported from the path given on the command line, its CPU
streaming path (``semi_crf_streaming_forward_pytorch`` /
``semi_crf_streaming_backward_pytorch`` via ``semi_crf_streaming_forward`` with
CPU tensors) and ``SemiMarkovCRFHead`` are run on small seeded inputs, and
inputs + outputs are written as plain arrays to ``tests/golden/*.npz``.  Only
those data files are used by the tests; nothing here runs on the GPU box.

What the fixtures pin that the exhaustive/closed-form checks cannot: the exact
fp32 rounding of the reference's forward/backward at medium T, the contents of
``ring_checkpoints``, the fp32 Viterbi table's tie-breaks in
``decode_with_traceback`` and the Python-float segment scores.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def make_inputs(B, T, K, C, seed, lengths=None, proj=False, dur_trans=False, centre=True):
    g = torch.Generator().manual_seed(seed)
    em = torch.randn(B, T, C, generator=g)
    if centre:
        em = em - em.mean(dim=1, keepdim=True)
    cum = torch.zeros(B, T + 1, C)
    cum[:, 1:] = torch.cumsum(em, dim=1)
    if dur_trans:
        trans = 0.1 * torch.randn(K, C, C, generator=g)
    else:
        trans = 0.1 * torch.randn(C, C, generator=g)
    db = 0.1 * torch.randn(K, C, generator=g)
    if lengths is None:
        lengths = torch.full((B,), T, dtype=torch.long)
    else:
        lengths = torch.tensor(lengths, dtype=torch.long)
    ps = pe = None
    if proj:
        ps = 0.1 * torch.randn(B, T, C, generator=g)
        pe = 0.1 * torch.randn(B, T, C, generator=g)
    return cum, trans, db, lengths, ps, pe


def streaming_case(ref, name, B, T, K, C, seed, semiring="log", grad_output=None, **kw):
    from torch_semimarkov.streaming.pytorch_reference import semi_crf_streaming_forward_pytorch

    cum, trans, db, lengths, ps, pe = make_inputs(B, T, K, C, seed, **kw)
    part_raw, ckpts, S = semi_crf_streaming_forward_pytorch(
        cum, trans, db, lengths, K, semiring, ps, pe
    )
    cum_r = cum.clone().requires_grad_(True)
    tr_r = trans.clone().requires_grad_(True)
    db_r = db.clone().requires_grad_(True)
    ps_r = ps.clone().requires_grad_(True) if ps is not None else None
    pe_r = pe.clone().requires_grad_(True) if pe is not None else None
    part = ref.semi_crf_streaming_forward(
        cum_r, tr_r, db_r, lengths, K, semiring=semiring, proj_start=ps_r, proj_end=pe_r,
        use_triton=False,
    )
    g = torch.ones(B) if grad_output is None else torch.tensor(grad_output, dtype=torch.float32)
    part.backward(g)
    out = dict(
        cum=cum.numpy(), transition=trans.numpy(), duration_bias=db.numpy(),
        lengths=lengths.numpy(), K=np.int64(K), semiring=np.array(semiring),
        grad_output=g.numpy(), partition=part.detach().numpy(),
        partition_raw=part_raw.numpy(), ring_checkpoints=ckpts.numpy(),
        checkpoint_interval=np.int64(S),
        grad_cum=cum_r.grad.numpy(), grad_transition=tr_r.grad.numpy(),
        grad_duration_bias=db_r.grad.numpy(),
    )
    if ps is not None:
        out.update(proj_start=ps.numpy(), proj_end=pe.numpy(),
                   grad_proj_start=ps_r.grad.numpy(), grad_proj_end=pe_r.grad.numpy())
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **out)
    print(f"wrote {name}: partition={part.detach().numpy()}")


def head_case(ref, name, C, K, H, B, T, lengths, seed, max_traceback_length=10000):
    torch.manual_seed(seed)
    head = ref.SemiMarkovCRFHead(num_classes=C, max_duration=K, hidden_dim=H)
    hidden = torch.randn(B, T, H if H is not None else C)
    lengths_t = torch.tensor(lengths, dtype=torch.long)
    labels = torch.randint(0, C, (B, T))
    loss = head.compute_loss(hidden, lengths_t, labels, use_triton=False, reduction="none")
    loss.sum().backward()
    with torch.no_grad():
        part = head(hidden, lengths_t, use_triton=False)["partition"]
        vit = head.decode(hidden, lengths_t, use_triton=False)
        res = head.decode_with_traceback(hidden, lengths_t, max_traceback_length)
    segs = []
    for b, sl in enumerate(res.segments):
        for s in sl:
            segs.append((b, s.start, s.end, s.label, s.score))
    seg_arr = np.array([[b, s, e, l] for (b, s, e, l, _) in segs], dtype=np.int64).reshape(-1, 4)
    seg_score = np.array([x for (*_, x) in segs], dtype=np.float64)
    out = dict(
        hidden=hidden.numpy(), lengths=lengths_t.numpy(), labels=labels.numpy(),
        transition=head.transition.detach().numpy(),
        duration_bias=head.duration_bias.detach().numpy(),
        loss=loss.detach().numpy(), partition=part.numpy(), viterbi=vit.numpy(),
        traceback_scores=res.scores.numpy(), segments=seg_arr, segment_scores=seg_score,
        grad_transition=head.transition.grad.numpy(),
        grad_duration_bias=head.duration_dist.duration_bias.grad.numpy(),
        C=np.int64(C), K=np.int64(K), max_traceback_length=np.int64(max_traceback_length),
    )
    if H is not None:
        out.update(proj_weight=head.projection.weight.detach().numpy(),
                   proj_bias=head.projection.bias.detach().numpy(),
                   grad_proj_weight=head.projection.weight.grad.numpy(),
                   grad_proj_bias=head.projection.bias.grad.numpy())
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **out)
    print(f"wrote {name}: loss={loss.detach().numpy()}, n_segments={len(segs)}")


def main(src):
    sys.path.insert(0, src)
    import torch_semimarkov as ref

    torch.set_num_threads(1)
    streaming_case(ref, "stream_basic", 2, 30, 5, 4, 101, grad_output=[0.5, 2.0])
    streaming_case(ref, "stream_varlen", 4, 50, 6, 3, 102, lengths=[50, 40, 30, 20])
    streaming_case(ref, "stream_k1", 2, 20, 1, 3, 103)
    streaming_case(ref, "stream_c24", 2, 50, 8, 24, 104)
    streaming_case(ref, "stream_t1", 2, 1, 4, 3, 105)
    streaming_case(ref, "stream_t2", 2, 2, 4, 3, 106)
    streaming_case(ref, "stream_proj", 2, 40, 6, 4, 107, proj=True, lengths=[40, 33])
    streaming_case(ref, "stream_durtrans", 2, 30, 5, 3, 108, dur_trans=True)
    streaming_case(ref, "stream_max", 3, 40, 6, 4, 109, semiring="max", lengths=[40, 31, 12])
    streaming_case(ref, "stream_nocentre", 2, 60, 7, 5, 110, centre=False)
    streaming_case(ref, "stream_medium", 1, 2000, 50, 8, 111)
    head_case(ref, "head_small", C=4, K=8, H=None, B=2, T=20, lengths=[20, 15], seed=201)
    head_case(ref, "head_proj", C=6, K=12, H=16, B=3, T=64, lengths=[64, 50, 9], seed=202)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src")
