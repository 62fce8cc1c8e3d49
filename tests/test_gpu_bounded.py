"""GPU parity of the bounded-memory (checkpointed) forward / backward
(``tsm_forward_checkpointed`` / ``tsm_backward_checkpointed``): the forward
keeps only per-window checkpoints, the backward recomputes alpha one window at
a time, top window first.  Its log partition and gradients are checked against
the fp64 oracle (log Z within 1e-5 relative, gradients within 1e-5 relative +
1e-4 absolute) and against the full-table backward of the same plan, over
several windows, lengths that end inside, exactly at and just past a window
edge, projections, narrow and wide label mixes and durations that take the
register and the atomic duration sums.
"""

import numpy as np
import pytest
import torch

from conftest import gpu_available
from oracle import cref
from oracle import streaming_ref as R

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0) if gpu_available() else None

import torch_semimarkov_amd as tsa  # noqa: E402,F401
from torch_semimarkov_amd import _native as N  # noqa: E402
from torch_semimarkov_amd.streaming import ops  # noqa: E402

RTOL_Z = 1e-5
GRAD_TOL = dict(rtol=1e-5, atol=1e-4)


def problem(B, T, K, C, seed, proj=False):
    g = torch.Generator().manual_seed(seed)
    sc = torch.randn(B, T, C, generator=g)
    cum = torch.zeros(B, T + 1, C, dtype=torch.float64)
    cum[:, 1:] = torch.cumsum(sc.double(), dim=1)
    cum = cum - cum.mean(dim=1, keepdim=True)  # centred, as the head builds it
    tr = 0.3 * torch.randn(C, C, generator=g)
    db = 0.3 * torch.randn(K, C, generator=g)
    ps = 0.5 * torch.randn(B, T, C, generator=g) if proj else None
    pe = 0.5 * torch.randn(B, T, C, generator=g) if proj else None
    return cum, tr, db, ps, pe


def chunk_len(B, T, C, K, proj):
    # a budget nothing fits gives the shortest window: one chunk
    w, _, _, _ = ops.checkpoint_plan(B, T, C, K, proj, proj, budget_bytes=1)
    return w


def run_ck(cum, tr, db, L, K, ps, pe, window, gout):
    B, Tp1, C = cum.shape
    T = Tp1 - 1
    nw = -(-T // window)
    d = lambda x: None if x is None else x.float().to(DEV).contiguous()
    c, t, b, p, e = d(cum), d(tr), d(db), d(ps), d(pe)
    Ld = L.to(DEV)
    part, z2, st, lv, ah, al = ops.scan_forward_ck(c, t, b, Ld, K, p, e, window, nw)
    g = ops.scan_backward_ck(c, t, b, Ld, K, p, e, window, st, lv, ah, al, z2, gout.to(DEV).contiguous())
    out = [x.cpu() for x in g[:3]]
    if ps is not None:
        out += [g[3].cpu(), g[4].cpu()]
    return part.cpu(), out


def run_full(cum, tr, db, L, K, ps, pe, gout):
    d = lambda x: None if x is None else x.float().to(DEV).contiguous()
    c, t, b, p, e = d(cum), d(tr), d(db), d(ps), d(pe)
    Ld = L.to(DEV)
    part, z2, ah, al, _ = ops.scan_forward(c, t, b, Ld, K, N.TSM_SEMIRING_LOG, p, e, True)
    g = ops.scan_backward(c, t, b, Ld, K, N.TSM_SEMIRING_LOG, p, e, ah, al, z2, gout.to(DEV).contiguous())
    out = [x.cpu() for x in g[:3]]
    if ps is not None:
        out += [g[3].cpu(), g[4].cpu()]
    return part.cpu(), out


def oracle(cum, tr, db, L, K, ps, pe, gout):
    if ps is None:
        res = cref.backward(cum, tr.double(), db.double(), L, K)
        w = gout.double().numpy()
        return res["logZ"], [res["grad_cum"] * w[:, None, None],
                             (res["grad_transition"] * w[:, None, None]).sum(0),
                             (res["grad_duration_bias"] * w[:, None, None]).sum(0)]
    c = cum.clone().requires_grad_(True)
    dd = lambda x: x.double().requires_grad_(True)
    t64, b64, p64, e64 = dd(tr), dd(db), dd(ps), dd(pe)
    z = R.streaming_oracle(c, t64, b64, L, K, "log", p64, e64)
    grads = torch.autograd.grad((z * gout.double()).sum(), [c, t64, b64, p64, e64])
    return z.detach().numpy(), [x.numpy() for x in grads]


NAMES = ("cum", "transition", "duration_bias", "proj_start", "proj_end")

# B, T, K, C, projections, window in chunks, lengths as fractions / offsets of the window
CASES = [
    (2, 3000, 40, 24, False, 1, "mixed"),
    (3, 2500, 12, 6, False, 2, "edges"),
    (2, 2200, 30, 16, True, 1, "mixed"),
    (2, 2600, 20, 64, False, 1, "edges"),
    (1, 5000, 200, 8, False, 3, "full"),
    (1, 4200, 400, 4, False, 2, "full"),
    (2, 1800, 2, 10, False, 1, "edges"),
]


def lengths_for(kind, B, T, window):
    if kind == "full":
        return [T] * B
    if kind == "mixed":
        return [T, T - window // 2 - 7][:B]
    # ends inside the first window, exactly at a window edge, just past one
    return [T, window, window + 1][:B]


@pytest.mark.parametrize("B,T,K,C,proj,wc,kind", CASES)
def test_checkpointed_backward_vs_oracle_and_full_table(B, T, K, C, proj, wc, kind):
    lc = chunk_len(B, T, C, K, proj)
    window = wc * lc
    nw = -(-T // window)
    assert nw >= 2, (lc, window, T)
    print(f"bounded B={B} T={T} K={K} C={C} proj={proj} Lc={lc} window={window} windows={nw}", flush=True)
    cum, tr, db, ps, pe = problem(B, T, K, C, 500 + K + C, proj)
    L = torch.tensor(lengths_for(kind, B, T, window), dtype=torch.long)
    gout = torch.linspace(1.0, 0.5, B)
    part, grads = run_ck(cum, tr, db, L, K, ps, pe, window, gout)
    z, want = oracle(cum, tr, db, L, K, ps, pe, gout)
    np.testing.assert_allclose(part.double().numpy(), z, rtol=RTOL_Z)
    for got, ref, name in zip(grads, want, NAMES):
        np.testing.assert_allclose(got.double().numpy(), ref, **GRAD_TOL, err_msg=name)
    # the full-table backward of the same inputs: the same quantities, other chunking and
    # other roundings (each within the bar of the oracle above, so within twice it of each other)
    pf, gf = run_full(cum, tr, db, L, K, ps, pe, gout)
    np.testing.assert_allclose(part.numpy(), pf.numpy(), rtol=2e-6)
    for got, ref, name in zip(grads, gf, NAMES):
        np.testing.assert_allclose(got.numpy(), ref.numpy(), rtol=2e-5, atol=5e-5, err_msg=name)


def test_checkpointed_window_aligned_with_sequence_end():
    """T a multiple of the window: the last checkpoint slot is not written past its end."""
    B, K, C = 2, 16, 8
    T = next(t for t in range(3000, 6000) if t % (2 * chunk_len(B, t, C, K, False)) == 0
             and t // chunk_len(B, t, C, K, False) >= 4)
    lc = chunk_len(B, T, C, K, False)
    cum, tr, db, _, _ = problem(B, T, K, C, 7)
    L = torch.tensor([T, 2 * lc])
    gout = torch.ones(B)
    part, grads = run_ck(cum, tr, db, L, K, None, None, 2 * lc, gout)
    z, want = oracle(cum, tr, db, L, K, None, None, gout)
    np.testing.assert_allclose(part.double().numpy(), z, rtol=RTOL_Z)
    for got, ref, name in zip(grads, want, NAMES):
        np.testing.assert_allclose(got.double().numpy(), ref, **GRAD_TOL, err_msg=name)


def test_checkpoint_plan_budget_and_memory():
    """A budget picks the longest window whose backward workspace fits it; the
    checkpointed pair needs far less device memory than the full tables."""
    B, T, K, C = 1, 200000, 30, 24
    w_all, nw_all, _, bw_all = ops.checkpoint_plan(B, T, C, K, False, False, budget_bytes=1 << 40)
    assert nw_all == 1
    budget = bw_all // 6
    w, nw, fw, bw = ops.checkpoint_plan(B, T, C, K, False, False, budget_bytes=budget)
    assert bw <= budget and nw >= 6 and w % chunk_len(B, T, C, K, False) == 0
    cum, tr, db, _, _ = problem(B, T, K, C, 3)
    L = torch.tensor([T])
    gout = torch.ones(B)
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    part, grads = run_ck(cum, tr, db, L, K, None, None, w, gout)
    peak_ck = torch.cuda.max_memory_allocated() - base
    torch.cuda.empty_cache()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    pf, gf = run_full(cum, tr, db, L, K, None, None, gout)
    peak_full = torch.cuda.max_memory_allocated() - base
    print(f"peak device memory: checkpointed {peak_ck / 2**20:.1f} MiB, full tables {peak_full / 2**20:.1f} MiB",
          flush=True)
    # inputs and outputs (cum, grad_cum) are common to both; the tables are not
    assert peak_ck < 0.6 * peak_full
    np.testing.assert_allclose(part.numpy(), pf.numpy(), rtol=2e-6)
    for got, ref, name in zip(grads, gf, NAMES):
        np.testing.assert_allclose(got.numpy(), ref.numpy(), rtol=2e-5, atol=5e-5, err_msg=name)


def test_checkpointed_rejects_bad_window_and_unsupported_plans():
    B, T, K, C = 1, 3000, 20, 8
    lc = chunk_len(B, T, C, K, False)
    with pytest.raises(ValueError, match="multiple of the chunk length"):
        ops._ck_workspace(B, T, C, K, False, False, lc + 1)
    with pytest.raises(NotImplementedError):
        ops.checkpoint_plan(B, T, 200, K, False, False)  # C > 64: no 16-lane fused plan


def test_streaming_forward_memory_budget_autograd():
    """semi_crf_streaming_forward(memory_budget=...) takes the checkpointed pair
    and gives the gradients of the full-table path; problems without a bounded
    plan (C > 64) keep the full tables."""
    B, T, K, C = 2, 3000, 24, 12
    cum, tr, db, ps, pe = problem(B, T, K, C, 21, proj=True)
    L = torch.tensor([T, 2100])
    outs = []
    for budget in (None, 0):
        x = [v.float().to(DEV).requires_grad_(True) for v in (cum, tr, db, ps, pe)]
        z = tsa.semi_crf_streaming_forward(x[0], x[1], x[2], L.to(DEV), K, proj_start=x[3], proj_end=x[4],
                                           memory_budget=budget)
        assert (type(z.grad_fn).__name__ == "SemiCRFStreamingCheckpointedHIPBackward") == (budget is not None)
        g = torch.autograd.grad((z * torch.tensor([1.0, 0.25], device=DEV)).sum(), x)
        outs.append((z.detach().cpu(), [v.cpu() for v in g]))
    np.testing.assert_allclose(outs[1][0].numpy(), outs[0][0].numpy(), rtol=2e-6)
    for got, ref, name in zip(outs[1][1], outs[0][1], NAMES):
        np.testing.assert_allclose(got.numpy(), ref.numpy(), rtol=2e-5, atol=5e-5, err_msg=name)
    C2 = 80
    c2 = torch.randn(1, 200, C2).cumsum(1).to(DEV).requires_grad_(True)
    z = tsa.semi_crf_streaming_forward(c2, torch.zeros(C2, C2, device=DEV), torch.zeros(8, C2, device=DEV),
                                       torch.tensor([200], device=DEV), 8, memory_budget=0)
    assert type(z.grad_fn).__name__ == "SemiCRFStreamingHIPBackward"
