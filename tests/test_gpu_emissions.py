"""GPU parity of the emission-input path: the scan, its gradients, the Viterbi
and the gold-path score computed from the projected scores (B, T, C)
(``tsm_*_emissions``), whose register-resident kernels carry the prefix sums
themselves, against the fp64 oracle run on ``cum = [0, cumsum(scores)]``.

The score gradient is the suffix sum of the cumulative-score gradient,
``d/dscores[t] = sum_{u > t} d/dcum[u]`` (for grad_output = 1 the posterior
occupancy of label c at position t); its expected values are built that way
from the oracle's ``grad_cum``.  Tolerances are the path's bar: log Z within
1e-5 relative, gradients within 1e-5 relative + 1e-4 absolute, Viterbi scores
within 1e-5 of the fp64 optimum with the optimum's segmentation on
gap-separated inputs.
"""

import numpy as np
import pytest
import torch

from conftest import gpu_available
from oracle import cref
from oracle import streaming_ref as R

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0) if gpu_available() else None

import torch_semimarkov_amd as tsa  # noqa: E402
from torch_semimarkov_amd import _native as N  # noqa: E402
from torch_semimarkov_amd.streaming import ops  # noqa: E402

RTOL_Z = 1e-5
GRAD_TOL = dict(rtol=1e-5, atol=1e-4)


def problem(B, T, K, C, seed, lengths=None, proj=False, tscale=0.3, dscale=0.3):
    g = torch.Generator().manual_seed(seed)
    sc = torch.randn(B, T, C, generator=g)
    tr = tscale * torch.randn(C, C, generator=g)
    db = dscale * torch.randn(K, C, generator=g)
    L = torch.full((B,), T, dtype=torch.long) if lengths is None else torch.tensor(lengths, dtype=torch.long)
    ps = 0.5 * torch.randn(B, T, C, generator=g) if proj else None
    pe = 0.5 * torch.randn(B, T, C, generator=g) if proj else None
    return sc, tr, db, L, ps, pe


def cum64(sc):
    c = torch.zeros(sc.shape[0], sc.shape[1] + 1, sc.shape[2], dtype=torch.float64)
    c[:, 1:] = torch.cumsum(sc.double(), dim=1)
    return c


def suffix(grad_cum):
    """d/dscores[t] = sum_{u > t} d/dcum[u] (numpy, (B, T+1, C) -> (B, T, C))."""
    g = np.asarray(grad_cum)[:, 1:]
    return np.ascontiguousarray(np.flip(np.cumsum(np.flip(g, 1), 1), 1))


def hip_emissions(sc, tr, db, L, K, ps=None, pe=None, semiring="log"):
    ins = [x.to(DEV).clone().requires_grad_(True) for x in (sc, tr, db, ps, pe) if x is not None]
    it = iter(ins)
    s, t, b = next(it), next(it), next(it)
    p = next(it) if ps is not None else None
    e = next(it) if pe is not None else None
    part = tsa.semi_crf_emissions_forward(s, t, b, L, K, semiring=semiring, proj_start=p, proj_end=e)
    grads = torch.autograd.grad(part.sum(), ins)
    return part.detach().cpu(), [x.cpu() for x in grads]


# B, T, K, C, lengths, environment, projections, plan entries the case must exercise
CASES = [
    (3, 300, 12, 6, [300, 177, 1], {}, False, {"fast": 1}),
    (2, 2000, 40, 24, [2000, 1500], {"TSM_FAST_J": "16"}, False, {"fast": 1, "mfused": 1}),
    (2, 2000, 40, 24, [2000, 1500], {"TSM_MARGINAL_PATH": "separate"}, False, {"fast": 1, "mfast": 1}),
    (1, 2400, 300, 24, None, {"TSM_SCAN_CHUNKS": "dual"}, False, {"fast": 1}),
    (2, 600, 16, 40, [600, 350], {}, True, {"fast": 1}),
    (2, 900, 9, 64, [900, 613], {}, False, {"fast": 1}),
    (2, 600, 20, 80, [600, 411], {}, False, {"fast": 0}),          # cooperative / generic: cum built first
    (2, 500, 9, 5, [500, 33], {"TSM_SCAN_PATH": "generic"}, False, {"fast": 0}),
]


@pytest.mark.parametrize("B,T,K,C,lengths,env,proj,plan", CASES)
def test_emissions_forward_backward_vs_fp64_oracle(B, T, K, C, lengths, env, proj, plan, monkeypatch):
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    info = N.plan_info(B, T, C, K, proj, proj)
    for k, v in plan.items():
        assert info[k] == v, (k, info)
    sc, tr, db, L, ps, pe = problem(B, T, K, C, 1000 + C + K, lengths, proj)
    part, grads = hip_emissions(sc, tr, db, L, K, ps, pe)
    if proj:
        c = cum64(sc).requires_grad_(True)
        d = lambda x: x.double().requires_grad_(True)
        t64, b64, p64, e64 = d(tr), d(db), d(ps), d(pe)
        want = R.streaming_oracle(c, t64, b64, L, K, "log", p64, e64)
        gc, gt, gd, gp, ge = torch.autograd.grad(want.sum(), [c, t64, b64, p64, e64])
        np.testing.assert_allclose(part.double().numpy(), want.detach().numpy(), rtol=RTOL_Z)
        ref = [suffix(gc.numpy()), gt.numpy(), gd.numpy(), gp.numpy(), ge.numpy()]
    else:
        res = cref.backward(cum64(sc), tr.double(), db.double(), L, K)
        np.testing.assert_allclose(part.double().numpy(), res["logZ"], rtol=RTOL_Z)
        ref = [suffix(res["grad_cum"]), res["grad_transition"].sum(0), res["grad_duration_bias"].sum(0)]
    for got, want, name in zip(grads, ref, ("scores", "transition", "duration_bias", "proj_start", "proj_end")):
        np.testing.assert_allclose(got.double().numpy(), want, **GRAD_TOL, err_msg=name)


@pytest.mark.parametrize("env", [{"TSM_MARGINAL_PATH": "separate"}, {"TSM_FAST_J": "16"}])
def test_emissions_long_sequence_coverage_pass(env, monkeypatch):
    """T = 70000: the coverage passes (block scales of the separate marginals,
    chunk factors of the fused backward) run on the score input."""
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    B, T, K, C = 1, 70000, 8, 4
    sc, tr, db, L, _, _ = problem(B, T, K, C, 77)
    part, grads = hip_emissions(sc, tr, db, L, K)
    res = cref.backward(cum64(sc), tr.double(), db.double(), L, K)
    np.testing.assert_allclose(part.double().numpy(), res["logZ"], rtol=RTOL_Z)
    ref = [suffix(res["grad_cum"]), res["grad_transition"].sum(0), res["grad_duration_bias"].sum(0)]
    for got, want, name in zip(grads, ref, ("scores", "transition", "duration_bias")):
        np.testing.assert_allclose(got.double().numpy(), want, **GRAD_TOL, err_msg=name)


def test_emissions_grad_output_weighting():
    """The score gradient is scaled per sequence by grad_output (zero isolates)."""
    B, T, K, C = 3, 800, 10, 12
    sc, tr, db, L, _, _ = problem(B, T, K, C, 5)
    w = torch.tensor([0.5, 0.0, 2.0])
    s = sc.to(DEV).requires_grad_(True)
    part = tsa.semi_crf_emissions_forward(s, tr.to(DEV), db.to(DEV), L, K)
    (gs,) = torch.autograd.grad((part * w.to(DEV)).sum(), [s])
    res = cref.backward(cum64(sc), tr.double(), db.double(), L, K)
    want = suffix(res["grad_cum"]) * w.double().numpy()[:, None, None]
    np.testing.assert_allclose(gs.cpu().double().numpy(), want, **GRAD_TOL)
    assert torch.all(gs[1] == 0)


def test_emissions_max_semiring_gradients_vs_oracle():
    """The max semiring with gradients (soft max-marginals) builds cum in the
    workspace and matches the fp64 oracle's max-semiring backward."""
    B, T, K, C = 2, 60, 6, 5
    sc, tr, db, L, _, _ = problem(B, T, K, C, 9, [60, 41])
    part, grads = hip_emissions(sc, tr, db, L, K, semiring="max")
    c = cum64(sc).requires_grad_(True)
    t64, b64 = tr.double().requires_grad_(True), db.double().requires_grad_(True)
    want = R.streaming_oracle(c, t64, b64, L, K, "max")
    gc, gt, gd = torch.autograd.grad(want.sum(), [c, t64, b64])
    np.testing.assert_allclose(part.double().numpy(), want.detach().numpy(), rtol=RTOL_Z)
    for got, ref in zip(grads, (suffix(gc.numpy()), gt.numpy(), gd.numpy())):
        np.testing.assert_allclose(got.double().numpy(), ref, **GRAD_TOL)


@pytest.mark.parametrize("alg", [N.TSM_VITERBI_AUTO, N.TSM_VITERBI_FACTORISED, N.TSM_VITERBI_EXACT])
def test_emissions_viterbi_vs_fp64_optimum(alg):
    """Viterbi on scores: within 1e-5 of the fp64 optimum, with its segments (the
    inputs are made gap-separated by a self-transition penalty).  EXACT builds cum
    with the prologue and is bit-identical to the exact kernel on that cum."""
    B, T, K, C = 2, 3000, 16, 12
    sc, tr, db, L, _, _ = problem(B, T, K, C, 31, [3000, 2111], tscale=0.5, dscale=0.5)
    tr = tr - 30.0 * torch.eye(C)
    if alg == N.TSM_VITERBI_AUTO:
        assert N.plan_info(B, T, C, K)["P"] >= 2
    args = [sc.to(DEV), tr.to(DEV), db.to(DEV), L.to(DEV), K, None, None, True, alg]
    score, cnt, segs = ops.viterbi_em(*args)
    c64 = cum64(sc)
    v64 = cref.viterbi(c64, tr.double(), db.double(), L, K, dtype=np.float64)
    np.testing.assert_allclose(score.cpu().double().numpy(), v64["score"], rtol=1e-5)
    cnt, segs = cnt.cpu(), segs.cpu()
    for b in range(B):
        got = [tuple(int(v) for v in segs[b, i]) for i in range(int(cnt[b]) - 1, -1, -1)]
        assert [s[:3] for s in got] == [tuple(s[:3]) for s in v64["segments"][b]], b
    if alg == N.TSM_VITERBI_EXACT:
        cum = tsa.emission_cum_scores(sc.to(DEV))
        s2, c2, g2 = ops.viterbi(cum, tr.to(DEV), db.to(DEV), L.to(DEV), K, None, None, True, alg)
        assert torch.equal(score.cpu(), s2.cpu()) and torch.equal(cnt, c2.cpu())


def test_emissions_no_grad_paths_and_decode():
    """No-grad log partition and Viterbi score through semi_crf_emissions_forward,
    and the head's decode / compute_loss against the cumulative-score path."""
    B, T, K, C = 2, 1500, 20, 8
    sc, tr, db, L, _, _ = problem(B, T, K, C, 11, [1500, 999])
    with torch.no_grad():
        z = tsa.semi_crf_emissions_forward(sc.to(DEV), tr.to(DEV), db.to(DEV), L, K)
        m = tsa.semi_crf_emissions_forward(sc.to(DEV), tr.to(DEV), db.to(DEV), L, K, semiring="max")
    c64 = cum64(sc)
    np.testing.assert_allclose(z.cpu().double().numpy(), cref.forward(c64, tr.double(), db.double(), L, K),
                               rtol=RTOL_Z)
    np.testing.assert_allclose(m.cpu().double().numpy(),
                               cref.forward(c64, tr.double(), db.double(), L, K, "max"), rtol=1e-5)


def test_gold_score_emissions_vs_oracle():
    """Gold-path score on scores: the fp64 oracle's score on cum (rtol 1e-6);
    d/dscores = grad_output * one-hot of the label inside the length; the shared
    gradients equal the cumulative-score kernel's."""
    B, T, K, C = 3, 700, 12, 7
    sc, tr, db, L, _, _ = problem(B, T, K, C, 13, [700, 350, 1])
    g = torch.Generator().manual_seed(3)
    labels = torch.randint(0, C, (B, T // 10 + 1), generator=g).repeat_interleave(10, dim=1)[:, :T].contiguous()
    w = torch.tensor([1.5, -0.5, 2.0])
    s = sc.to(DEV).requires_grad_(True)
    t, d = tr.to(DEV).requires_grad_(True), db.to(DEV).requires_grad_(True)
    gold = tsa.score_gold_emissions(s, labels.to(DEV), L.to(DEV), t, d, K)
    gs, gt, gd = torch.autograd.grad((gold * w.to(DEV)).sum(), [s, t, d])
    want = R.score_gold(cum64(sc), labels, L, tr.double(), db.double(), K)
    np.testing.assert_allclose(gold.detach().cpu().double().numpy(), want.numpy(), rtol=1e-6, atol=1e-5)
    onehot = torch.nn.functional.one_hot(labels, C).double() * (torch.arange(T)[None, :] < L[:, None])[..., None]
    np.testing.assert_allclose(gs.cpu().double().numpy(), (onehot * w.double()[:, None, None]).numpy())
    c = tsa.emission_cum_scores(sc.to(DEV)).requires_grad_(True)
    t2, d2 = tr.to(DEV).requires_grad_(True), db.to(DEV).requires_grad_(True)
    gold2 = tsa.score_gold_vectorized(c, labels.to(DEV), L.to(DEV), t2, d2, K)
    gt2, gd2 = torch.autograd.grad((gold2 * w.to(DEV)).sum(), [t2, d2])
    assert torch.equal(gt.cpu(), gt2.cpu()) and torch.equal(gd.cpu(), gd2.cpu())


def test_head_compute_loss_vs_fp64():
    """compute_loss (scores straight to the kernels) against the fp64 oracle of the
    same head (fp64 projection, cumsum, partition and gold score): the loss and
    the transition / duration-bias / projection-weight gradients at the path's
    bar.  The projection-bias gradient of label c is the difference of two
    occupancy sums of about B*T/C; fp32 storage of the per-position sums already
    moves it by ~1e-5 of that scale, so its tolerance is scaled by the occupancy
    (as in the cfg1 head test).  The reference's composition (forward()'s
    partition minus score_gold_vectorized on its cum_scores) is held to the same
    bar."""
    torch.manual_seed(0)
    C, K, H = 10, 24, 32
    head = tsa.SemiMarkovCRFHead(C, K, hidden_dim=H).to(DEV)
    B, T = 3, 900
    h = torch.randn(B, T, H, device=DEV)
    L = torch.tensor([900, 640, 77])
    labels = torch.randint(0, C, (B, T), device=DEV)
    params = list(head.parameters())
    loss = head.compute_loss(h, L.to(DEV), labels, reduction="sum")
    g_em = torch.autograd.grad(loss, params)
    res = head(h, L.to(DEV))
    loss2 = (res["partition"] - tsa.score_gold_vectorized(res["cum_scores"], labels, L.to(DEV), head.transition,
                                                           head.duration_bias, K)).sum()
    g_cum = torch.autograd.grad(loss2, params)
    # fp64 oracle
    W = head.projection.weight.detach().double().cpu()
    bl = head.projection.bias.detach().double().cpu()
    tr = head.transition.detach().double().cpu()
    db = head.duration_bias.detach().double().cpu()
    h64 = h.double().cpu()
    sc = h64 @ W.T + bl
    c64 = cum64(sc)
    ref = cref.backward(c64, tr, db, L, K)
    c_g = c64.clone().requires_grad_(True)
    t_g, d_g = tr.clone().requires_grad_(True), db.clone().requires_grad_(True)
    gold = R.score_gold(c_g, labels.cpu(), L, t_g, d_g, K)
    gcg, gtg, gdg = torch.autograd.grad(gold.sum(), [c_g, t_g, d_g])
    d_sc = torch.from_numpy(suffix(ref["grad_cum"] - gcg.numpy()))
    want = {
        "loss": float(ref["logZ"].sum() - gold.sum().item()),
        "transition": ref["grad_transition"].sum(0) - gtg.numpy(),
        "duration": ref["grad_duration_bias"].sum(0) - gdg.numpy(),
        "weight": torch.einsum("btc,bth->ch", d_sc, h64).numpy(),
        "bias": d_sc.sum((0, 1)).numpy(),
    }
    occ = (np.arange(T + 1)[None, :, None] * ref["grad_cum"]).sum((0, 1))
    names = {id(head.transition): "transition", id(head.projection.weight): "weight",
             id(head.projection.bias): "bias"}
    for got_loss, grads in ((loss, g_em), (loss2, g_cum)):
        np.testing.assert_allclose(got_loss.item(), want["loss"], rtol=1e-5)
        for prm, g in zip(params, grads):
            name = names.get(id(prm), "duration")
            g = g.cpu().double().numpy()
            if name == "bias":
                tol = 1e-4 + 1e-5 * np.maximum(np.abs(want["bias"]), np.abs(occ))
                assert np.all(np.abs(g - want["bias"]) <= tol), (np.abs(g - want["bias"]) / tol).max()
            else:
                np.testing.assert_allclose(g, want[name], rtol=1e-5, atol=2e-4, err_msg=name)


def test_emissions_c_abi_refuses_empty_sequences():
    lib = N.lib()
    import ctypes

    n = ctypes.c_size_t(0)
    assert lib.tsm_forward_emissions_workspace(1, 0, 4, 3, 0, 0, 0, 0, ctypes.byref(n)) == 1
    with pytest.raises(ValueError, match="T >= 1"):
        tsa.semi_crf_emissions_forward(torch.zeros(1, 0, 4, device=DEV), torch.zeros(4, 4, device=DEV),
                                       torch.zeros(3, 4, device=DEV), torch.zeros(1, dtype=torch.long), 3)
