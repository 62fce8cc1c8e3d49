"""GPU parity tests: the HIP path (through the C ABI) against the oracle and the
reference's golden vectors.

Tolerances (the path's stated parity bar): log Z within 1e-5 relative; gradients
within 1e-5 relative + 1e-4 absolute against the fp64 oracle; Viterbi scores and
segmentations bit-exact against the fp32 restatement of the reference.
"""

import numpy as np
import pytest
import torch

from conftest import gpu_available, load_golden
from oracle import brute as BR
from oracle import streaming_ref as R

pytestmark = pytest.mark.gpu

if gpu_available():
    DEV = torch.device("cuda", 0)
else:  # collected on CPU, never run there
    DEV = None

import torch_semimarkov_amd as tsa  # noqa: E402
from torch_semimarkov_amd import _native as N  # noqa: E402
from torch_semimarkov_amd.streaming import launch_streaming_hip_backward, launch_streaming_hip_kernel, ops  # noqa: E402

RTOL_Z = 1e-5
GRAD_TOL = dict(rtol=1e-5, atol=1e-4)

STREAM_FIXTURES = [
    "stream_basic", "stream_varlen", "stream_k1", "stream_c24", "stream_t1", "stream_t2",
    "stream_proj", "stream_max", "stream_nocentre", "stream_medium", "stream_durtrans",
]


def fixture_inputs(z, requires_grad=False):
    t = lambda k: torch.from_numpy(z[k]).to(DEV)
    cum, tr, db = t("cum"), t("transition"), t("duration_bias")
    L = torch.from_numpy(z["lengths"])
    ps = t("proj_start") if "proj_start" in z else None
    pe = t("proj_end") if "proj_end" in z else None
    if requires_grad:
        for x in (cum, tr, db, ps, pe):
            if x is not None:
                x.requires_grad_(True)
    return cum, tr, db, L, int(z["K"]), str(z["semiring"]), ps, pe


def rand_problem(B, T, K, C, seed, lengths=None, proj=False, centre=False, tscale=0.1, dscale=0.1):
    g = torch.Generator().manual_seed(seed)
    em = torch.randn(B, T, C, generator=g)
    if centre:
        em = em - em.mean(1, keepdim=True)
    cum = torch.zeros(B, T + 1, C)
    cum[:, 1:] = em.cumsum(1)
    tr = tscale * torch.randn(C, C, generator=g)
    db = dscale * torch.randn(K, C, generator=g)
    L = torch.full((B,), T, dtype=torch.long) if lengths is None else torch.tensor(lengths, dtype=torch.long)
    ps = 0.1 * torch.randn(B, T, C, generator=g) if proj else None
    pe = 0.1 * torch.randn(B, T, C, generator=g) if proj else None
    return cum, tr, db, L, ps, pe


def oracle_fp64(cum, tr, db, L, K, semiring="log", ps=None, pe=None, g=None):
    """fp64 oracle partition and grads (weighted by g)."""
    d = lambda x: None if x is None else x.detach().cpu().double().requires_grad_(True)
    c64, t64, b64, p64, e64 = d(cum), d(tr), d(db), d(ps), d(pe)
    part = R.streaming_oracle(c64, t64, b64, L.cpu(), K, semiring, p64, e64)
    gw = torch.ones_like(part) if g is None else g.double().cpu()
    ins = [x for x in (c64, t64, b64, p64, e64) if x is not None]
    grads = torch.autograd.grad((part * gw).sum(), ins)
    return part.detach(), grads


def to_dev(*xs):
    return [None if x is None else x.to(DEV) for x in xs]


def run_hip(cum, tr, db, L, K, semiring="log", ps=None, pe=None, g=None):
    cum, tr, db, ps, pe = to_dev(cum, tr, db, ps, pe)
    ins = [x.clone().requires_grad_(True) for x in (cum, tr, db, ps, pe) if x is not None]
    it = iter(ins)
    c, t, b = next(it), next(it), next(it)
    p = next(it) if ps is not None else None
    e = next(it) if pe is not None else None
    part = tsa.semi_crf_streaming_forward(c, t, b, L, K, semiring=semiring, proj_start=p, proj_end=e)
    gw = torch.ones_like(part) if g is None else g.to(DEV)
    grads = torch.autograd.grad((part * gw).sum(), ins)
    return part.detach().cpu(), [x.cpu() for x in grads]


@pytest.fixture(params=["fast", "generic"])
def scan_path(request, monkeypatch):
    """Run a test on the register-resident log-semiring scan (where the plan
    allows it) and again with TSM_SCAN_PATH=generic on the generic kernels."""
    if request.param == "generic":
        monkeypatch.setenv("TSM_SCAN_PATH", "generic")
    else:
        monkeypatch.delenv("TSM_SCAN_PATH", raising=False)
    return request.param


def assert_grads(got, want, tol=GRAD_TOL):
    for a, b in zip(got, want):
        np.testing.assert_allclose(a.double().numpy(), b.double().numpy(), **tol)


# --------------------------------------------------------------------------- golden vectors
@pytest.mark.parametrize("name", STREAM_FIXTURES)
def test_forward_backward_match_reference_golden(name, scan_path):
    z = load_golden(name)
    cum, tr, db, L, K, sr, ps, pe = fixture_inputs(z, requires_grad=True)
    part = tsa.semi_crf_streaming_forward(cum, tr, db, L, K, semiring=sr, proj_start=ps, proj_end=pe)
    want = torch.from_numpy(z["partition"])
    np.testing.assert_allclose(part.detach().cpu().numpy(), want.numpy(), rtol=RTOL_Z, atol=1e-5)
    g = torch.from_numpy(z["grad_output"]).to(DEV)
    (part * g).sum().backward()
    got = [cum.grad.cpu(), tr.grad.cpu(), db.grad.cpu()] + ([ps.grad.cpu(), pe.grad.cpu()] if ps is not None else [])
    ref32 = [torch.from_numpy(z[k]) for k in ("grad_cum", "grad_transition", "grad_duration_bias")]
    if ps is not None:
        ref32 += [torch.from_numpy(z["grad_proj_start"]), torch.from_numpy(z["grad_proj_end"])]
    if float(np.abs(z["partition"]).max()) < 1000:
        # short sequences: the reference's fp32 gradients are accurate to ~1e-5
        assert_grads(got, ref32)
    else:
        # |alpha| ~ 5e3: the reference's raw fp32 log-space values lose ~1e-3 in the
        # marginals, so the yardstick is the fp64 oracle; the build must also be
        # closer to it than the reference is
        _, g64 = oracle_fp64(*(torch.from_numpy(z[k]) for k in ("cum", "transition", "duration_bias")),
                             torch.from_numpy(z["lengths"]), K, sr, g=torch.from_numpy(z["grad_output"]))
        assert_grads(got, g64)
        for a, r, w in zip(got, ref32, g64):
            assert (a.double() - w).abs().max() <= (r.double() - w).abs().max()


@pytest.mark.parametrize("name", STREAM_FIXTURES)
def test_inference_matches_reference_golden(name):
    """No-grad path: log partition within tolerance; the max semiring bit-exact with
    the exact Viterbi kernel, and within 1e-5 on the default path (AUTO: the
    factorised scan when the plan cuts a sequence into several chunks)."""
    z = load_golden(name)
    cum, tr, db, L, K, sr, ps, pe = fixture_inputs(z)
    with torch.no_grad():
        part = tsa.semi_crf_streaming_forward(cum, tr, db, L, K, semiring=sr, proj_start=ps, proj_end=pe)
        vit = tsa.semi_crf_streaming_forward(cum, tr, db, L, K, semiring="max", proj_start=ps, proj_end=pe)
        exact, _, _ = ops.viterbi(cum, tr, db, L.to(DEV), K, ps, pe, False, N.TSM_VITERBI_EXACT)
    np.testing.assert_allclose(part.cpu().numpy(), z["partition_raw"], rtol=RTOL_Z, atol=1e-5)
    want_max, _, _ = R.forward(*[torch.from_numpy(z[k]) for k in ("cum", "transition", "duration_bias", "lengths")],
                               K, "max",
                               torch.from_numpy(z["proj_start"]) if "proj_start" in z else None,
                               torch.from_numpy(z["proj_end"]) if "proj_end" in z else None)
    assert torch.equal(exact.cpu(), want_max)
    np.testing.assert_allclose(vit.cpu().double().numpy(), want_max.double().numpy(), rtol=1e-5, atol=1e-5)
    if sr == "max":
        np.testing.assert_allclose(part.cpu().double().numpy(), z["partition_raw"], rtol=1e-5, atol=1e-5)


# --------------------------------------------------------------------------- (K, C, C) transitions
def rand_trans3(rows, C, seed, scale=0.3):
    g = torch.Generator().manual_seed(seed)
    return scale * torch.randn(rows, C, C, generator=g)


# B, T, K, C, lengths, proj, semiring, expected plan entries.  Together they cover
# 4 / 16 / 64 lanes per label, transitions in LDS and in global memory, label
# groups with several destination labels (C = 40) and several source labels per
# lane (C = 70) in the marginal kernel, projections and the max semiring.
DURTRANS_CASES = [
    (2, 30, 5, 4, [30, 17], False, "log", dict(DJ=4, dtrl=1)),
    (2, 50, 9, 3, [50, 50], True, "log", dict(DJ=4)),
    (2, 45, 12, 6, [45, 30], False, "max", dict(DJ=16)),
    (2, 40, 40, 5, [40, 33], True, "log", dict(DJ=64)),
    (1, 60, 10, 40, None, False, "log", dict(DJ=16, DG=64)),
    (1, 40, 6, 70, None, True, "log", dict(DJ=4, DG=64)),
    (1, 80, 60, 24, None, False, "log", dict(DJ=16, dtrl=0)),
    (3, 28, 7, 4, [28, 6, 0], False, "log", dict()),
]


@pytest.mark.parametrize("B,T,K,C,lengths,proj,sr,plan", DURTRANS_CASES)
def test_duration_dependent_transitions_vs_fp64_oracle(B, T, K, C, lengths, proj, sr, plan):
    got = N.plan_info(B, T, C, K, proj, proj, trans_rows=K)
    assert got["dense"] == 1
    for key, v in plan.items():
        assert got[key] == v, (key, got)
    cum, _, db, L, ps, pe = rand_problem(B, T, K, C, 4000 + T + K + C, lengths, proj)
    tr = rand_trans3(K, C, 17 + C)
    g = torch.linspace(0.5, 2.0, B)
    p64, g64 = oracle_fp64(cum, tr, db, L, K, sr, ps, pe, g)
    part, grads = run_hip(cum, tr, db, L, K, sr, ps, pe, g)
    np.testing.assert_allclose(part.double().numpy(), p64.numpy(), rtol=RTOL_Z, atol=1e-6)
    assert grads[1].shape == (K, C, C)
    assert_grads(grads, g64)


def test_duration_dependent_transitions_chunked_vs_fp64_oracle():
    """Long sequences: the dense scans run chunked, speculative and verified."""
    B, T, K, C = 2, 3000, 8, 6
    assert N.plan_info(B, T, C, K, trans_rows=K)["P"] > 1
    cum, _, db, L, _, _ = rand_problem(B, T, K, C, 4242, [3000, 2200])
    tr = rand_trans3(K, C, 99)
    g = torch.tensor([1.0, 0.5])
    p64, g64 = oracle_fp64(cum, tr, db, L, K, "log", g=g)
    cum_d, tr_d, db_d = to_dev(cum, tr, db)
    out = ops.scan_forward(cum_d, tr_d, db_d, L.to(DEV), K, N.TSM_SEMIRING_LOG, None, None, True)
    assert int(out[4].sum()) == 0  # every speculative chunk verified
    part, grads = run_hip(cum, tr, db, L, K, "log", g=g)
    np.testing.assert_allclose(part.double().numpy(), p64.numpy(), rtol=RTOL_Z)
    assert_grads(grads, g64)


def test_duration_dependent_transitions_k1_and_extra_matrices():
    """K = 1 uses duration 1 and so transition[1] (a 2-matrix table): the same
    problem as the static transition transition[1].  Matrices no duration uses
    (index 0, and indices beyond max(K-1, 1)) get zero gradients."""
    B, T, C = 2, 40, 5
    cum, tr2, db, L, _, _ = rand_problem(B, T, 1, C, 808, [40, 29])
    tr3 = torch.stack([torch.randn(C, C), tr2, torch.randn(C, C)])  # 3 matrices, only [1] used
    p2, g2 = run_hip(cum, tr2, db, L, 1)
    p3, g3 = run_hip(cum, tr3, db, L, 1)
    np.testing.assert_allclose(p3.numpy(), p2.numpy(), rtol=1e-6)
    np.testing.assert_allclose(g3[1][1].numpy(), g2[1].numpy(), rtol=1e-5, atol=1e-6)
    assert torch.all(g3[1][0] == 0) and torch.all(g3[1][2] == 0)
    for a, b in ((g3[0], g2[0]), (g3[2], g2[2])):
        np.testing.assert_allclose(a.numpy(), b.numpy(), rtol=1e-5, atol=1e-6)
    with pytest.raises(ValueError, match="duration-dependent transition"):
        tsa.semi_crf_streaming_forward(cum.to(DEV), tr3[:1].to(DEV), db.to(DEV), L, 1)


def test_duration_dependent_transitions_viterbi_exact():
    """Inference in the max semiring with (K, C, C) transitions: the exact kernel,
    bit-identical to the reference's fp32 recursion, with the segmentation of its
    traceback; the factorised algorithm is refused."""
    B, T, K, C = 3, 90, 8, 5
    cum, _, db, L, _, _ = rand_problem(B, T, K, C, 515, [90, 61, 4], tscale=0.5, dscale=0.5)
    tr = rand_trans3(K, C, 23, scale=0.8)
    args = to_dev(cum, tr, db, L) + [K, None, None, True]
    score, cnt, segs = ops.viterbi(*args, N.TSM_VITERBI_AUTO)
    want, _, _ = R.forward(cum, tr, db, L, K, "max")
    assert torch.equal(score.cpu(), want)
    with torch.no_grad():
        vit = tsa.semi_crf_streaming_forward(*to_dev(cum, tr, db), L, K, semiring="max")
    assert torch.equal(vit.cpu(), want)
    for b in range(B):
        ref_segs, _ = R.viterbi_traceback_single(cum[b], tr, db, K, int(L[b]))
        got = [tuple(int(v) for v in segs[b, i]) for i in range(int(cnt[b]) - 1, -1, -1)]
        assert got == [tuple(s) for s in ref_segs]
    with pytest.raises(NotImplementedError, match="static"):
        ops.viterbi(*args, N.TSM_VITERBI_FACTORISED)


# --------------------------------------------------------------------------- fp64 oracle
CASES = [
    # B, T, K, C, lengths, proj, semiring
    (2, 40, 6, 4, [40, 23], False, "log"),
    (3, 35, 1, 5, [35, 20, 1], False, "log"),
    (2, 50, 9, 3, [50, 50], True, "log"),
    (1, 64, 12, 33, None, False, "log"),
    (2, 30, 5, 1, [30, 12], False, "log"),
    (2, 45, 7, 4, [45, 30], False, "max"),
    (4, 25, 30, 6, [25, 24, 3, 0], False, "log"),
    (2, 40, 9, 12, [40, 33], True, "log"),      # 32-lane label groups
    (2, 36, 5, 16, [36, 20], False, "max"),
    (1, 30, 4, 70, None, False, "log"),         # 4-lane groups
    # unit durations (Kmax = 1): the position-parallel marginal kernel
    (3, 70, 2, 5, [70, 41, 1], True, "log"),
    (2, 90, 1, 16, [90, 64], True, "max"),
    (2, 300, 1, 3, [300, 299], False, "log"),
]

# Plans outside the register / LDS-ring fast path: more than 32 durations per
# lane (batched online log-sum-exp, duration bias from LDS) and rings too large
# for LDS (global-memory rings, the C=128 configuration's path).
SLOW_PATH_CASES = [
    (2, 600, 2200, 2, [600, 433], False, "log", dict(RMAX=0, global_rings=0)),
    (2, 700, 560, 20, [700, 615], False, "log", dict(RMAX=0, global_rings=1)),
    (1, 200, 64, 128, None, False, "log", dict(RMAX=0, global_rings=1)),
    (2, 120, 40, 128, [120, 77], True, "max", dict(RMAX=0, global_rings=1)),
]


@pytest.mark.parametrize("B,T,K,C,lengths,proj,sr,plan", SLOW_PATH_CASES)
def test_generic_scan_paths_vs_fp64_oracle(B, T, K, C, lengths, proj, sr, plan, monkeypatch):
    monkeypatch.setenv("TSM_SCAN_PATH", "generic")
    got = N.plan_info(B, T, C, K, proj, proj)
    for key, v in plan.items():
        assert got[key] == v, (key, got)
    cum, tr, db, L, ps, pe = rand_problem(B, T, K, C, 3000 + T + K + C, lengths, proj)
    g = torch.linspace(0.5, 2.0, B)
    p64, g64 = oracle_fp64(cum, tr, db, L, K, sr, ps, pe, g)
    part, grads = run_hip(cum, tr, db, L, K, sr, ps, pe, g)
    np.testing.assert_allclose(part.double().numpy(), p64.numpy(), rtol=RTOL_Z, atol=1e-6)
    assert_grads(grads, g64)


# Cooperative scans (rings too large for one CU): groups of CG blocks, CCL labels
# each, exchanging their row of results every step.
COOP_CASES = [
    (2, 300, 40, 128, [300, 177], False, dict(CG=4, CR=8)),
    (2, 240, 40, 128, [240, 0], True, dict(CG=4, CR=8)),
    (1, 150, 300, 128, None, False, dict(CG=8, CR=24)),
    (1, 80, 500, 128, None, True, dict(CG=8, CR=32)),   # the C=128, K=500 configuration's instance
    (1, 300, 200, 96, None, False, dict(CG=4, CR=16)),
    (3, 200, 9, 80, [200, 150, 7], True, dict(CG=4, CR=8)),
]


@pytest.mark.parametrize("B,T,K,C,lengths,proj,plan", COOP_CASES)
def test_coop_scan_vs_fp64_oracle(B, T, K, C, lengths, proj, plan):
    got = N.plan_info(B, T, C, K, proj, proj)
    assert got["coop"] == 1 and got["fast"] == 0, got
    for key, v in plan.items():
        assert got[key] == v, (key, got)
    cum, tr, db, L, ps, pe = rand_problem(B, T, K, C, 4000 + T + K + C, lengths, proj)
    g = torch.linspace(0.5, 2.0, B)
    p64, g64 = oracle_fp64(cum, tr, db, L, K, "log", ps, pe, g)
    part, grads = run_hip(cum, tr, db, L, K, "log", ps, pe, g)
    live = L > 0
    np.testing.assert_allclose(part[live].double().numpy(), p64[live].numpy(), rtol=RTOL_Z, atol=1e-6)
    assert_grads(grads, g64)


def test_coop_scan_chunked_vs_fp64_oracle():
    """Several speculative chunks per sequence on the cooperative scan."""
    B, T, K, C = 2, 4000, 12, 72
    got = N.plan_info(B, T, C, K)
    assert got["coop"] == 1 and got["P"] > 1, got
    cum, tr, db, L, _, _ = rand_problem(B, T, K, C, 4321, [4000, 2900])
    p64, g64 = oracle_fp64(cum, tr, db, L, K)
    part, grads = run_hip(cum, tr, db, L, K)
    np.testing.assert_allclose(part.double().numpy(), p64.numpy(), rtol=RTOL_Z)
    assert_grads(grads, g64)


def test_coop_scan_recomputes_non_mixing_chunks():
    """Sticky transitions on the cooperative scan: speculative chunks fail
    verification and the group recomputes them in the sequential repair pass."""
    B, T, K, C = 1, 2400, 5, 72
    assert N.plan_info(B, T, C, K)["coop"] == 1
    g = torch.Generator().manual_seed(6)
    em = 0.01 * torch.randn(B, T, C, generator=g)
    em[:, :50, 0] += 2.0
    cum = torch.zeros(B, T + 1, C)
    cum[:, 1:] = em.cumsum(1)
    tr = torch.full((C, C), -40.0)
    tr.fill_diagonal_(0.0)
    db = torch.zeros(K, C)
    L = torch.tensor([T])
    with torch.no_grad():
        _, _, _, _, rec = ops.scan_forward(cum.to(DEV), tr.to(DEV), db.to(DEV), L.to(DEV), K, 0, None, None, False)
    assert int(rec.sum()) > 0
    p64, g64 = oracle_fp64(cum, tr, db, L, K)
    part, grads = run_hip(cum, tr, db, L, K)
    np.testing.assert_allclose(part.double().numpy(), p64.numpy(), rtol=RTOL_Z)
    assert_grads(grads, g64)


COOP_MAX_CASES = [
    (2, 300, 40, 128, [300, 177], False),
    (3, 200, 9, 80, [200, 150, 7], True),
    (1, 300, 200, 96, None, False),
]


@pytest.mark.parametrize("B,T,K,C,lengths,proj", COOP_MAX_CASES)
def test_coop_max_semiring_vs_fp64_oracle(B, T, K, C, lengths, proj):
    """The max-plus cooperative scan (forward and beta) under the max semiring's
    gradients (soft max-marginals) against the fp64 oracle."""
    assert N.plan_info(B, T, C, K, proj, proj)["coop"] == 1
    cum, tr, db, L, ps, pe = rand_problem(B, T, K, C, 4500 + T + K + C, lengths, proj)
    g = torch.linspace(0.5, 2.0, B)
    p64, g64 = oracle_fp64(cum, tr, db, L, K, "max", ps, pe, g)
    part, grads = run_hip(cum, tr, db, L, K, "max", ps, pe, g)
    live = L > 0
    np.testing.assert_allclose(part[live].double().numpy(), p64[live].numpy(), rtol=RTOL_Z, atol=1e-6)
    assert_grads(grads, g64)


@pytest.mark.parametrize("proj", [False, True])
def test_coop_factorised_viterbi_vs_fp64_optimum(proj):
    """C = 96 (cooperative plan, several chunks per sequence): AUTO takes the
    factorised max-plus cooperative scan; its score is within 1e-5 of the fp64
    optimum and its segments are the optimum's on gap-separated inputs (a
    self-transition penalty removes runs of one label cut into segments)."""
    from oracle import cref

    B, T, K, C = 2, 6000, 12, 96
    info = N.plan_info(B, T, C, K, proj, proj)
    assert info["coop"] == 1 and info["P"] >= 2, info
    cum, tr, db, L, ps, pe = rand_problem(B, T, K, C, 4700, [6000, 4333], proj, tscale=0.5, dscale=0.5)
    tr = tr - 30.0 * torch.eye(C)
    args = [cum.to(DEV), tr.to(DEV), db.to(DEV), L.to(DEV), K] + to_dev(ps, pe)
    score, cnt, segs = ops.viterbi(*args, True, N.TSM_VITERBI_AUTO)
    f_score, _, _ = ops.viterbi(*args, True, N.TSM_VITERBI_FACTORISED)
    assert torch.equal(score.cpu(), f_score.cpu())
    if ps is None:
        v64 = cref.viterbi(cum.double(), tr.double(), db.double(), L, K, dtype=np.float64)
        np.testing.assert_allclose(score.cpu().double().numpy(), v64["score"], rtol=1e-5)
        cnt, segs = cnt.cpu(), segs.cpu()
        for b in range(B):
            got = [tuple(int(v) for v in segs[b, i]) for i in range(int(cnt[b]) - 1, -1, -1)]
            assert [x[:3] for x in got] == [tuple(x[:3]) for x in v64["segments"][b]], b
    else:
        # projections: the fp64 max-semiring oracle's value
        want = R.streaming_oracle(cum.double(), tr.double(), db.double(), L, K, "max", ps.double(), pe.double())
        np.testing.assert_allclose(score.cpu().double().numpy(), want.numpy(), rtol=1e-5)
    e_score, _, _ = ops.viterbi(*args, True, N.TSM_VITERBI_EXACT)
    np.testing.assert_allclose(score.cpu().numpy(), e_score.cpu().numpy(), rtol=2e-5)


def test_coop_factorised_viterbi_long_durations_c128():
    """The C = 128, K = 500 cooperative instance (32 durations per lane, the
    C = 128 configuration's) with backpointers: score within 1e-5 of the fp64
    optimum and the optimum's segments; the exact kernel cannot hold this ring
    in LDS, so before the max-plus cooperative scan this Viterbi was refused."""
    from oracle import cref

    B, T, K, C = 1, 1000, 500, 128
    info = N.plan_info(B, T, C, K)
    assert info["coop"] == 1 and info["CR"] == 32, info
    g = torch.Generator().manual_seed(4800)
    cum = torch.zeros(B, T + 1, C)
    cum[:, 1:] = (0.2 * torch.randn(B, T, C, generator=g)).cumsum(1)
    tr = 0.5 * torch.randn(C, C, generator=g) - 30.0 * torch.eye(C)
    k = torch.arange(K, dtype=torch.float32)[:, None]
    db = -0.5 * ((k - 150.0) / 50.0) ** 2 + 0.1 * torch.randn(K, C, generator=g)  # durations around 150
    L = torch.tensor([T])
    score, cnt, segs = ops.viterbi(cum.to(DEV), tr.to(DEV), db.to(DEV), L.to(DEV), K, None, None, True,
                                   N.TSM_VITERBI_AUTO)
    v64 = cref.viterbi(cum.double(), tr.double(), db.double(), L, K, dtype=np.float64)
    np.testing.assert_allclose(score.cpu().double().numpy(), v64["score"], rtol=1e-5)
    got = [tuple(int(v) for v in segs[0, i].cpu()) for i in range(int(cnt[0]) - 1, -1, -1)]
    assert [x[:3] for x in got] == [tuple(x[:3]) for x in v64["segments"][0]]
    assert max(x[1] - x[0] + 1 for x in got) > 64  # durations beyond the first lanes' ranges occur


@pytest.mark.parametrize("B,T,K,C,lengths,proj,sr", CASES)
def test_random_problems_vs_fp64_oracle(B, T, K, C, lengths, proj, sr, scan_path):
    cum, tr, db, L, ps, pe = rand_problem(B, T, K, C, 1000 + T + K + C, lengths, proj)
    g = torch.linspace(0.5, 2.0, B)
    p64, g64 = oracle_fp64(cum, tr, db, L, K, sr, ps, pe, g)
    part, grads = run_hip(cum, tr, db, L, K, sr, ps, pe, g)
    live = L > 0
    np.testing.assert_allclose(part[live].double().numpy(), p64[live].numpy(), rtol=RTOL_Z, atol=1e-6)
    assert_grads(grads, g64)


@pytest.mark.parametrize("B,T,K,C,lengths,sr", [
    (2, 600, 20, 12, [600, 377], "log"),
    (3, 900, 40, 24, [900, 1, 512], "log"),
    (1, 1300, 100, 32, None, "log"),
    (2, 700, 30, 20, [700, 333], "max"),
    (2, 700, 1, 8, [700, 450], "log"),
    (2, 500, 1, 6, None, "max"),
])
def test_eight_lane_groups_vs_fp64_oracle(B, T, K, C, lengths, sr, monkeypatch):
    """Plans with few chunks take 16 lanes per label; TSM_FAST_J=8 keeps the 8-lane
    instances (several durations per lane, a four-source label mix at C > 16, the
    one-source mix of single-duration plans with C <= 8, the separate marginal
    kernel) checked against the fp64 oracle, with the Viterbi score of the 8-lane
    factorised scan against the exact kernel."""
    monkeypatch.delenv("TSM_SCAN_PATH", raising=False)
    monkeypatch.setenv("TSM_FAST_J", "8")
    info = N.plan_info(B, T, C, K)
    assert info["fast"] == 1 and info["FJ"] == 8 and info["mfused"] == 0, info
    cum, tr, db, L, _, _ = rand_problem(B, T, K, C, 808 + T + K, lengths)
    g = torch.linspace(0.5, 2.0, B)
    p64, g64 = oracle_fp64(cum, tr, db, L, K, sr, None, None, g)
    part, grads = run_hip(cum, tr, db, L, K, sr, None, None, g)
    np.testing.assert_allclose(part.double().numpy(), p64.numpy(), rtol=RTOL_Z, atol=1e-6)
    assert_grads(grads, g64)
    args = (cum.to(DEV), tr.to(DEV), db.to(DEV), L.to(DEV), K, None, None)
    f_score, _, _ = ops.viterbi(*args, False, N.TSM_VITERBI_FACTORISED)
    e_score, _, _ = ops.viterbi(*args, False, N.TSM_VITERBI_EXACT)
    np.testing.assert_allclose(f_score.cpu().numpy(), e_score.cpu().numpy(), rtol=2e-5)


@pytest.mark.parametrize("lengths", [[2600, 1900], [2600, 1560]])
def test_chunked_scan_vs_fp64_oracle(lengths, scan_path):
    """T long enough for several speculative chunks (warm-up + verification); the
    second case has lengths that are exact multiples of the chunk length (520)."""
    B, T, K, C = 2, 2600, 8, 4
    cum, tr, db, L, _, _ = rand_problem(B, T, K, C, 77, lengths=lengths)
    from torch_semimarkov_amd import _native as N

    assert N.plan_info(B, T, C, K)["P"] > 1
    p64, g64 = oracle_fp64(cum, tr, db, L, K)
    part, grads = run_hip(cum, tr, db, L, K)
    np.testing.assert_allclose(part.double().numpy(), p64.numpy(), rtol=RTOL_Z)
    assert_grads(grads, g64)


def test_verifier_recomputes_non_mixing_chunks(scan_path):
    """Sticky transitions keep early evidence alive across chunk boundaries, so
    the warmed-up states disagree with the exact ones and chunks are recomputed
    from the previous chunk's exact state; results still match the oracle."""
    B, T, K, C = 1, 2400, 5, 3
    g = torch.Generator().manual_seed(5)
    em = 0.01 * torch.randn(B, T, C, generator=g)
    em[:, :50, 0] += 2.0
    cum = torch.zeros(B, T + 1, C)
    cum[:, 1:] = em.cumsum(1)
    tr = torch.full((C, C), -40.0)
    tr.fill_diagonal_(0.0)
    db = torch.zeros(K, C)
    L = torch.tensor([T])
    with torch.no_grad():
        _, _, _, _, rec = ops.scan_forward(cum.to(DEV), tr.to(DEV), db.to(DEV), L.to(DEV), K, 0, None, None, False)
    assert int(rec.sum()) > 0
    p64, g64 = oracle_fp64(cum, tr, db, L, K)
    part, grads = run_hip(cum, tr, db, L, K)
    np.testing.assert_allclose(part.double().numpy(), p64.numpy(), rtol=RTOL_Z)
    assert_grads(grads, g64)


def test_speculation_threshold_within_gradient_bar(monkeypatch):
    """Slowly mixing input (self-transition bonus 4, weak emissions): after the
    warm-up, some speculative chunks' boundary spreads lie between the default
    acceptance threshold (4e-6 log2 units, set from the gradient bar: an
    accepted spread s moves a marginal by at most ~1.4 s relative) and 2e-4.
    With TSM_SPEC_TOL=2e-4 those chunks are accepted as they are, so the result
    differs from the default run, which runs them again; the default's partition
    and gradients are within the bar of the fp64 oracle."""
    from oracle import cref

    monkeypatch.delenv("TSM_SCAN_PATH", raising=False)
    B, T, C, K = 1, 8000, 6, 20
    g = torch.Generator().manual_seed(77)
    em = 0.3 * torch.randn(B, T, C, generator=g)
    cum = torch.zeros(B, T + 1, C)
    cum[:, 1:] = em.cumsum(1)
    tr = 4.0 * torch.eye(C) - 4.0 / C + 0.05 * torch.randn(C, C, generator=g)
    db = 0.1 * torch.randn(K, C, generator=g)
    L = torch.tensor([T])
    assert N.plan_info(B, T, C, K)["P"] > 8
    monkeypatch.setenv("TSM_SPEC_TOL", "2e-4")
    p_loose, g_loose = run_hip(cum, tr, db, L, K)
    monkeypatch.delenv("TSM_SPEC_TOL")
    part, grads = run_hip(cum, tr, db, L, K)
    assert any(not torch.equal(a, b) for a, b in zip(g_loose, grads)), "no spread landed in (4e-6, 2e-4]"
    ref = cref.backward(cum, tr, db, L, K)
    np.testing.assert_allclose(part.double().numpy(), ref["logZ"], rtol=RTOL_Z)
    for got, key in zip(grads, ("grad_cum", "grad_transition", "grad_duration_bias")):
        want = ref[key] if key == "grad_cum" else ref[key].sum(0)
        np.testing.assert_allclose(got.double().numpy(), want, **GRAD_TOL, err_msg=key)


def test_grad_output_weighting_and_isolation(scan_path):
    """tests/test_streaming_triton.py:901-1087: shared grads are sum_b g_b * grad_b, per-sequence
    grads are scaled, a zero weight isolates a sequence."""
    cum, tr, db, L, _, _ = rand_problem(2, 30, 5, 4, 9, [30, 22])
    _, ga = run_hip(cum, tr, db, L, 5, g=torch.tensor([1.0, 0.0]))
    _, gb = run_hip(cum, tr, db, L, 5, g=torch.tensor([0.0, 1.0]))
    _, gh = run_hip(cum, tr, db, L, 5, g=torch.tensor([0.5, 2.0]))
    assert torch.all(ga[0][1] == 0) and torch.all(gb[0][0] == 0)
    for i in range(3):
        torch.testing.assert_close(gh[i], 0.5 * ga[i] + 2.0 * gb[i], rtol=1e-5, atol=1e-6)


def test_deterministic_bitwise(scan_path):
    cum, tr, db, L, ps, pe = rand_problem(3, 300, 10, 6, 3, [300, 250, 10], proj=True)
    a = run_hip(cum, tr, db, L, 10, ps=ps, pe=pe)
    b = run_hip(cum, tr, db, L, 10, ps=ps, pe=pe)
    assert torch.equal(a[0], b[0])
    for x, y in zip(a[1], b[1]):
        assert torch.equal(x, y)


# Backward with the segment marginals fused into the 16-lane register-resident
# beta scan: plans with 16-lane groups (more than 32 labels, or more than 256
# durations).  Each chunk accumulates in its own frame; the finalize rescales.
FUSED_CASES = [
    # B, T, K, C, lengths, proj
    (2, 3000, 40, 40, [3000, 2211], False),       # several speculative chunks, ragged
    (1, 4000, 120, 36, None, True),                # projections
    (3, 1500, 300, 24, [1500, 650, 299], False),   # the headline's lane layout (19 durations per lane)
    (2, 6000, 280, 12, [6000, 4117], True),        # long durations, few labels, projections
    (1, 1800, 64, 64, None, False),                # 64 labels: 4096 transition pairs
    (2, 2080, 33, 48, [2080, 1040], False),        # lengths that are multiples of the chunk length
    (2, 700, 1, 40, [700, 333], False),            # one duration: every position is a boundary
    (1, 900, 2, 36, None, True),                   # K = 2 (one register per lane, 15 padded lanes)
]


def _fused_plan(B, T, C, K, proj):
    info = N.plan_info(B, T, C, K, proj, proj)
    assert info["mfused"] == 1 and info["FJ"] == 16, info
    return info


@pytest.mark.parametrize("B,T,K,C,lengths,proj", FUSED_CASES)
def test_fused_backward_vs_fp64_oracle(B, T, K, C, lengths, proj, monkeypatch):
    monkeypatch.delenv("TSM_SCAN_PATH", raising=False)
    monkeypatch.delenv("TSM_MARGINAL_PATH", raising=False)
    _fused_plan(B, T, C, K, proj)
    cum, tr, db, L, ps, pe = rand_problem(B, T, K, C, 5000 + T + K + C, lengths, proj)
    g = torch.linspace(0.5, 2.0, B)
    p64, g64 = oracle_fp64(cum, tr, db, L, K, "log", ps, pe, g)
    part, grads = run_hip(cum, tr, db, L, K, "log", ps, pe, g)
    np.testing.assert_allclose(part.double().numpy(), p64.numpy(), rtol=RTOL_Z)
    assert_grads(grads, g64)


def test_fused_backward_banded_transitions(monkeypatch):
    """Transitions of -1000 outside a band of width 3: the transition ranges
    exceed what the one-pass label mix and the factorised transition gradient
    accept, so both take their exact forms."""
    monkeypatch.delenv("TSM_SCAN_PATH", raising=False)
    monkeypatch.delenv("TSM_MARGINAL_PATH", raising=False)
    B, T, K, C = 2, 2000, 40, 36
    _fused_plan(B, T, C, K, False)
    cum, tr, db, L, _, _ = rand_problem(B, T, K, C, 4242, [2000, 1333])
    idx = torch.arange(C)
    tr[(idx[:, None] - idx[None, :]).abs() > 3] = -1000.0
    g = torch.tensor([1.0, 0.7])
    p64, g64 = oracle_fp64(cum, tr, db, L, K, g=g)
    part, grads = run_hip(cum, tr, db, L, K, g=g)
    np.testing.assert_allclose(part.double().numpy(), p64.numpy(), rtol=RTOL_Z)
    assert_grads(grads, g64)


def _ops_backward(cum, tr, db, L, K, ps=None, pe=None, g=None):
    """forward (storing alpha) + backward through the custom ops: grads and the
    backward's recomputed-chunk counts."""
    cum, tr, db, ps, pe = to_dev(cum, tr, db, ps, pe)
    Ld = L.to(DEV)
    with torch.no_grad():
        part, z2, ah, al, _ = ops.scan_forward(cum, tr, db, Ld, K, 0, ps, pe, True)
        gw = torch.ones_like(part) if g is None else g.to(DEV)
        gc, gt, gd, gps, gpe, rec = ops.scan_backward(cum, tr, db, Ld, K, 0, ps, pe, ah, al, z2, gw)
    return [x.cpu() for x in (gc, gt, gd, gps, gpe)], rec.cpu()


@pytest.mark.parametrize("drop", [30.0, 60.0, 1e9])
def test_fused_backward_suppressed_durations(drop, monkeypatch):
    """Some durations of some labels suppressed by a large negative bias (30 and
    60 nats below the rest, and the reference's NEG_INF = -1e9 masking): the
    duration sums are kept without each term's bias factor and multiplied by it
    when folded, so a lane whose factors fall below 2^-64 takes the exact
    two-pass form; the gradients match the fp64 oracle either way."""
    monkeypatch.delenv("TSM_SCAN_PATH", raising=False)
    monkeypatch.delenv("TSM_MARGINAL_PATH", raising=False)
    B, T, K, C = 2, 3000, 40, 40
    _fused_plan(B, T, C, K, False)
    cum, tr, db, L, _, _ = rand_problem(B, T, K, C, 5150, [3000, 1977])
    db[20:33, ::3] -= drop
    g = torch.tensor([1.0, 0.6])
    p64, g64 = oracle_fp64(cum, tr, db, L, K, g=g)
    part, grads = run_hip(cum, tr, db, L, K, g=g)
    np.testing.assert_allclose(part.double().numpy(), p64.numpy(), rtol=RTOL_Z)
    assert_grads(grads, g64)


def test_fused_backward_recomputes_non_mixing_chunks(monkeypatch):
    """Sticky transitions and evidence at the sequence end: the beta states of
    the speculative chunks disagree with the exact ones, chunks are recomputed
    (in parallel, then sequentially from the neighbour's state) and their fused
    marginals recomputed with them; gradients still match the oracle."""
    monkeypatch.delenv("TSM_SCAN_PATH", raising=False)
    monkeypatch.delenv("TSM_MARGINAL_PATH", raising=False)
    B, T, K, C = 1, 6000, 300, 20
    _fused_plan(B, T, C, K, False)
    g = torch.Generator().manual_seed(15)
    em = 0.01 * torch.randn(B, T, C, generator=g)
    em[:, -50:, 0] += 2.0
    cum = torch.zeros(B, T + 1, C)
    cum[:, 1:] = em.cumsum(1)
    tr = torch.full((C, C), -40.0)
    tr.fill_diagonal_(0.0)
    db = torch.zeros(K, C)
    L = torch.tensor([T])
    _, rec = _ops_backward(cum, tr, db, L, K)
    assert int(rec.sum()) > 0
    p64, g64 = oracle_fp64(cum, tr, db, L, K)
    part, grads = run_hip(cum, tr, db, L, K)
    np.testing.assert_allclose(part.double().numpy(), p64.numpy(), rtol=RTOL_Z)
    assert_grads(grads, g64)


@pytest.mark.parametrize("marginals", ["fused", "separate"])
def test_two_chunks_per_cu_vs_fp64_oracle(marginals, monkeypatch):
    """Scan directions whose kernels leave registers for a second workgroup on
    every SIMD run two chunks per CU, with shorter rings (compacted every 96
    steps here) and a chunk count of their own; the fused backward keeps one
    chunk per CU.  TSM_SCAN_CHUNKS=dual takes that chunking on a problem the
    oracle can check, with the headline's lane layout (C=24, 19 durations per
    lane): the forward in two chunks and, with separate marginals, the beta scan
    too."""
    monkeypatch.delenv("TSM_SCAN_PATH", raising=False)
    monkeypatch.setenv("TSM_SCAN_CHUNKS", "dual")
    if marginals == "separate":
        monkeypatch.setenv("TSM_MARGINAL_PATH", "separate")
    else:
        monkeypatch.delenv("TSM_MARGINAL_PATH", raising=False)
    B, T, K, C = 2, 2400, 300, 24
    info = N.plan_info(B, T, C, K)
    assert info["dualF"] == 1 and info["P2"] > info["P"], info
    assert 0 < info["regsF"] <= 128 and 2 * info["fast_lds2"] <= 160 * 1024, info
    if marginals == "separate":
        assert info["mfused"] == 0 and info["dualB"] == 1, info
    else:
        assert info["mfused"] == 1 and info["dualB"] == 0, info
    cum, tr, db, L, _, _ = rand_problem(B, T, K, C, 4242, [2400, 1333])
    g = torch.tensor([0.75, 1.5])
    p64, g64 = oracle_fp64(cum, tr, db, L, K, "log", None, None, g)
    part, grads = run_hip(cum, tr, db, L, K, "log", None, None, g)
    np.testing.assert_allclose(part.double().numpy(), p64.numpy(), rtol=RTOL_Z)
    assert_grads(grads, g64)


def test_two_chunks_per_cu_full_size_config3(monkeypatch):
    """At the headline size (B=1, T=10^6, C=24, K=300) the log forward runs two
    chunks per CU (its kernel fits in 128 VGPRs); its partition and alpha
    table match the plan with one chunk per CU (TSM_SCAN_CHUNKS=single) up to
    the speculative chunks' verification tolerance (2e-4 in log2 units)."""
    monkeypatch.delenv("TSM_SCAN_PATH", raising=False)
    monkeypatch.delenv("TSM_SCAN_CHUNKS", raising=False)
    B, T, C, K = 1, 1_000_000, 24, 300
    info = N.plan_info(B, T, C, K)
    assert info["dualF"] == 1 and info["P2"] == 2 * info["P"] and 0 < info["regsF"] <= 128, info
    g = torch.Generator().manual_seed(20261203)
    em = torch.randn(B, T, C, generator=g)
    tr = 0.1 * torch.randn(C, C, generator=g)
    db = 0.1 * torch.randn(K, C, generator=g)
    cum = torch.zeros(B, T + 1, C)
    cum[:, 1:] = torch.cumsum(em, dim=1)
    L = torch.full((B,), T, dtype=torch.long)
    args = [x.to(DEV) for x in (cum, tr, db, L)]
    with torch.no_grad():
        _, z2, ah, al, _ = ops.scan_forward(*args, K, 0, None, None, True)
        monkeypatch.setenv("TSM_SCAN_CHUNKS", "single")
        assert N.plan_info(B, T, C, K)["dualF"] == 0
        _, z1, bh, bl, _ = ops.scan_forward(*args, K, 0, None, None, True)
        np.testing.assert_allclose(z2.cpu().numpy(), z1.cpu().numpy(), rtol=RTOL_Z)
        d = ((ah.double() + al.unsqueeze(-1)) - (bh.double() + bl.unsqueeze(-1))).abs().max().item()
    assert d <= 1e-3, d


def test_fused_backward_full_size_config3(monkeypatch):
    """The headline configuration (B=1, T=10^6, C=24, K=300): the fused backward
    against the separate marginal kernel (itself checked against the oracle
    above), and the size-independent identities of the gradients: every
    segment has one duration and one incoming transition (sum grad_db = sum
    grad_transition = expected segment count) and one start and one end
    (grad_cum sums to zero)."""
    monkeypatch.delenv("TSM_SCAN_PATH", raising=False)
    B, T, C, K = 1, 1_000_000, 24, 300
    g = torch.Generator().manual_seed(20261203)
    em = torch.randn(B, T, C, generator=g)
    tr = 0.1 * torch.randn(C, C, generator=g)
    db = torch.zeros(K, C)
    db[1:] = -0.01 * torch.arange(1, K, dtype=torch.float32).unsqueeze(1) + 0.05 * torch.randn(K - 1, C, generator=g)
    cum = torch.zeros(B, T + 1, C)
    cum[:, 1:] = torch.cumsum(em, dim=1)
    L = torch.full((B,), T, dtype=torch.long)
    monkeypatch.delenv("TSM_MARGINAL_PATH", raising=False)
    _fused_plan(B, T, C, K, False)
    fused, _ = _ops_backward(cum, tr, db, L, K)
    monkeypatch.setenv("TSM_MARGINAL_PATH", "separate")
    assert N.plan_info(B, T, C, K)["mfused"] == 0
    sep, _ = _ops_backward(cum, tr, db, L, K)
    for a, b in zip(fused[:3], sep[:3]):
        np.testing.assert_allclose(a.double().numpy(), b.double().numpy(), **GRAD_TOL)
    gc, gt, gd = (x.double() for x in fused[:3])
    n_seg = gd.sum()
    assert 1000 < n_seg < T
    assert abs(gt.sum() - n_seg) <= 1e-5 * n_seg
    assert abs(gc.sum()) <= 1e-5 * gc.abs().sum()


def test_k1_full_size_config2_vs_hmm(scan_path):
    """Config 2 of the benchmark set (B=32, T=10^4, C=8, K=1) against a probability-space HMM in fp64."""
    B, T, C, K = 32, 10_000, 8, 1
    g = torch.Generator().manual_seed(20261202)
    em = torch.randn(B, T, C, generator=g)
    tr = 0.1 * torch.randn(C, C, generator=g)
    db = 0.1 * torch.randn(1, C, generator=g)
    cum = torch.zeros(B, T + 1, C)
    cum[:, 1:] = em.cumsum(1)
    L = torch.full((B,), T)
    part, grads = run_hip(cum, tr, db, L, K)
    cum64 = cum.double().numpy()
    for b in range(0, B, 8):
        logZ, state_post, trans_counts, _ = BR.hmm_forward_backward(cum64[b], tr.double().numpy(),
                                                                    db[0].double().numpy(), T)
        assert abs(part[b].item() - logZ) <= RTOL_Z * abs(logZ)
        want = np.zeros((T + 1, C))
        want[1:] += state_post
        want[:-1] -= state_post
        np.testing.assert_allclose(grads[0][b].double().numpy(), want, rtol=1e-5, atol=1e-4)


# --------------------------------------------------------------------------- exact Viterbi
def _path_total_fp64(cum_b, tr, db, K, n, segs):
    """Checks that ``segs`` (start, end, label, prev) tile [0, n) with durations
    1..K-1 and chained labels, and returns its fp64 score."""
    pos, total, prev = 0, 0.0, None
    for (s, e, c, cp) in segs:
        assert s == pos and s <= e and e - s + 1 <= max(K - 1, 1)
        if prev is not None:
            assert cp == prev
        total += R.segment_score(cum_b, tr, db, K, s, e, c, cp)
        pos, prev = e + 1, c
    assert pos == n
    return total


@pytest.mark.parametrize("B,T,K,C,lengths", [(3, 120, 10, 6, [120, 77, 5]), (2, 60, 1, 4, [60, 31]),
                                             (2, 3000, 12, 8, [3000, 2200]), (2, 900, 40, 24, [900, 0])])
@pytest.mark.parametrize("tie_free", [False, True])
def test_viterbi_factorised_vs_fp64_optimum(B, T, K, C, lengths, tie_free):
    """The factorised (chunked, verified) Viterbi: scores within 1e-5 of the fp64
    optimum and a valid segmentation whose fp64 score is that optimum.  Runs of
    one label tie exactly (durations of consecutive same-label segments can be
    permuted at equal total), so the segmentation itself is compared bit-exactly
    on tie-free inputs, where self-transitions are penalised out of every optimum.
    The multi-chunk case exercises speculation in the max semiring."""
    _viterbi_factorised_check(B, T, K, C, lengths, tie_free)


def test_viterbi_factorised_two_chunks_per_cu(monkeypatch):
    """The factorised Viterbi forward with two chunks per CU (shorter rings, its
    own chunk count; TSM_SCAN_CHUNKS=dual on a problem the oracle can check,
    with the headline's lane layout: C=24, 19 durations per lane): the same
    checks as above on tie-free inputs."""
    monkeypatch.setenv("TSM_SCAN_CHUNKS", "dual")
    B, T, K, C = 2, 2400, 300, 24
    info = N.plan_info(B, T, C, K)
    assert info["dualV"] == 1 and info["P2"] > info["P"] and 0 < info["regsV"] <= 128, info
    _viterbi_factorised_check(B, T, K, C, [2400, 1333], True)


def _viterbi_factorised_check(B, T, K, C, lengths, tie_free):
    cum, tr, db, L, _, _ = rand_problem(B, T, K, C, 57 + C, lengths, tscale=0.5, dscale=0.5)
    if tie_free:
        tr = tr - 30.0 * torch.eye(C)
    score, cnt, segs = ops.viterbi(cum.to(DEV), tr.to(DEV), db.to(DEV), L.to(DEV), K, None, None, True,
                                   N.TSM_VITERBI_FACTORISED)
    want, _, _ = R.forward(cum.double(), tr.double(), db.double(), L, K, "max")
    live = L > 0
    np.testing.assert_allclose(score.cpu()[live].double().numpy(), want[live].numpy(), rtol=1e-5)
    cnt = cnt.cpu()
    segs = segs.cpu()
    for b in range(B):
        n = int(L[b])
        got = [tuple(int(v) for v in segs[b, i]) for i in range(int(cnt[b]) - 1, -1, -1)]
        if n == 0:
            assert got == []
            continue
        total = _path_total_fp64(cum[b].double(), tr.double(), db.double(), K, n, got)
        assert abs(total - float(want[b])) <= 1e-5 * abs(float(want[b])) + 1e-6, b
        if tie_free:
            ref_segs, _ = R.viterbi_traceback_single(cum[b].double(), tr.double(), db.double(), K, n)
            assert got == [tuple(s) for s in ref_segs], b
    if T >= 3000:
        assert N.plan_info(B, T, C, K)["P"] > 1


@pytest.mark.parametrize("B,T,K,C,lengths", [(3, 150, 9, 5, [150, 64, 1]), (2, 1200, 16, 12, [1200, 700])])
def test_viterbi_factorised_with_projections(B, T, K, C, lengths):
    """Factorised Viterbi with proj_start / proj_end: scores within 1e-5 of the
    fp64 optimum, and on tie-free inputs the same segments as the exact kernel
    (the reference's fp32 operation order)."""
    cum, tr, db, L, ps, pe = rand_problem(B, T, K, C, 71 + C, lengths, proj=True, tscale=0.5, dscale=0.5)
    tr = tr - 30.0 * torch.eye(C)
    args = to_dev(cum, tr, db, L) + [K] + to_dev(ps, pe) + [True]
    s_f, c_f, g_f = ops.viterbi(*args, N.TSM_VITERBI_FACTORISED)
    s_e, c_e, g_e = ops.viterbi(*args, N.TSM_VITERBI_EXACT)
    want, _, _ = R.forward(cum.double(), tr.double(), db.double(), L, K, "max", ps.double(), pe.double())
    np.testing.assert_allclose(s_f.cpu().double().numpy(), want.numpy(), rtol=1e-5)
    assert torch.equal(c_f, c_e)
    for b in range(B):
        n = int(c_f[b])
        assert torch.equal(g_f[b, :n], g_e[b, :n]), b


def test_viterbi_auto_picks_factorised_for_large_problems():
    B, T, K, C = 2, 20000, 64, 32
    cum, tr, db, L, _, _ = rand_problem(B, T, K, C, 91, tscale=0.5, dscale=0.5)
    args = (cum.to(DEV), tr.to(DEV), db.to(DEV), L.to(DEV), K, None, None, True)
    s_auto, c_auto, g_auto = ops.viterbi(*args, N.TSM_VITERBI_AUTO)
    s_fact, c_fact, g_fact = ops.viterbi(*args, N.TSM_VITERBI_FACTORISED)
    s_ex, c_ex, g_ex = ops.viterbi(*args, N.TSM_VITERBI_EXACT)
    assert torch.equal(s_auto, s_fact) and torch.equal(c_auto, c_fact)
    for b in range(B):  # rows past the count are not written
        n = int(c_auto[b])
        assert torch.equal(g_auto[b, :n], g_fact[b, :n])
    # the exact algorithm accumulates raw fp32 path scores (|score| ~ 1e5 here): allow its drift
    np.testing.assert_allclose(s_fact.cpu().numpy(), s_ex.cpu().numpy(), rtol=5e-5)


# --------------------------------------------------------------------------- chunked backtrace
def _sticky_problem(B, T, K, C, lengths, winner, seed):
    """Label chains that never merge.  A self-transition bonus of +100 dwarfs every
    emission difference, so each label's best path stays in that label and is made
    of unit segments (two of them beat one of duration 2 by ~100); `winner` gains
    0.01 per position and is the optimum.  Walks that start at label 0 therefore
    never meet the true path, and every chunk below the top one is walked again
    from its true entry node."""
    g = torch.Generator().manual_seed(seed)
    em = 0.05 * torch.randn(B, T, C, generator=g)
    em[:, :, winner] += 0.01
    cum = torch.zeros(B, T + 1, C)
    cum[:, 1:] = em.cumsum(1)
    tr = torch.full((C, C), -5.0) + 105.0 * torch.eye(C)
    db = 0.1 * torch.randn(K, C, generator=g)
    db[1] = 0.0  # unit segments: no label gains on duration bias
    return cum, tr, db, torch.tensor(lengths, dtype=torch.long)


@pytest.mark.parametrize("algorithm", ["exact", "factorised"])
@pytest.mark.parametrize("walk", ["lds", "global"])
def test_backtrace_rewalks_chunks_that_never_merge(algorithm, walk, monkeypatch):
    """Chunked backtrace where no speculative walk merges: the result must still be
    the true path (unit segments of the winning label, every chunk's record full)."""
    if walk == "global":
        monkeypatch.setenv("TSM_BACKTRACE_PATH", "global")
    B, T, K, C, winner = 2, 5000, 6, 4, 2
    lengths = [5000, 3333]
    cum, tr, db, L = _sticky_problem(B, T, K, C, lengths, winner, 123)
    alg = N.TSM_VITERBI_EXACT if algorithm == "exact" else N.TSM_VITERBI_FACTORISED
    score, cnt, segs = ops.viterbi(*to_dev(cum, tr, db, L), K, None, None, True, alg)
    want, _, _ = R.forward(cum.double(), tr.double(), db.double(), L, K, "max")
    np.testing.assert_allclose(score.cpu().double().numpy(), want.numpy(), rtol=1e-5)
    cnt, segs = cnt.cpu(), segs.cpu()
    for b in range(B):
        n = lengths[b]
        assert int(cnt[b]) == n
        expect = torch.tensor([[t, t, winner, winner] for t in range(n - 1, -1, -1)], dtype=torch.int32)
        assert torch.equal(segs[b, :n], expect), b


@pytest.mark.parametrize("walk", ["lds", "global"])
def test_backtrace_many_chunks_vs_oracle(walk, monkeypatch):
    """Chunked backtrace on long random sequences (several chunks each, ragged):
    the exact algorithm's segments equal the fp32 restatement's traceback, and
    the factorised algorithm's path is a valid segmentation at the fp64 optimum."""
    if walk == "global":
        monkeypatch.setenv("TSM_BACKTRACE_PATH", "global")
    B, T, K, C = 3, 6000, 12, 8
    lengths = [6000, 4500, 2100]
    cum, tr, db, L, _, _ = rand_problem(B, T, K, C, 202, lengths, tscale=0.5, dscale=0.5)
    args = to_dev(cum, tr, db, L) + [K, None, None, True]
    s_e, c_e, g_e = ops.viterbi(*args, N.TSM_VITERBI_EXACT)
    s_f, c_f, g_f = ops.viterbi(*args, N.TSM_VITERBI_FACTORISED)
    want, _, _ = R.forward(cum.double(), tr.double(), db.double(), L, K, "max")
    np.testing.assert_allclose(s_f.cpu().double().numpy(), want.numpy(), rtol=1e-5)
    c_e, g_e, c_f, g_f = c_e.cpu(), g_e.cpu(), c_f.cpu(), g_f.cpu()
    for b in range(B):
        n = lengths[b]
        ref, _ = R.viterbi_traceback_single(cum[b], tr, db, K, n)
        got = [tuple(int(v) for v in g_e[b, i]) for i in range(int(c_e[b]) - 1, -1, -1)]
        assert got == [tuple(s) for s in ref], b
        fact = [tuple(int(v) for v in g_f[b, i]) for i in range(int(c_f[b]) - 1, -1, -1)]
        total = _path_total_fp64(cum[b].double(), tr.double(), db.double(), K, n, fact)
        assert abs(total - float(want[b])) <= 1e-5 * abs(float(want[b])) + 1e-6, b


# --------------------------------------------------------------------------- emission prologue
PROLOGUE_CASES = [(2, 37, 5, torch.float32), (3, 1000, 24, torch.float32), (1, 700, 300, torch.float32),
                  (2, 513, 8, torch.bfloat16), (2, 257, 6, torch.float16), (1, 1, 3, torch.float32)]


@pytest.mark.parametrize("B,T,C,dtype", PROLOGUE_CASES)
@pytest.mark.parametrize("centre", [False, True])
def test_emission_prologue_vs_fp64(B, T, C, dtype, centre):
    """Cumulative scores = the fp32 rounding of the fp64 prefix sums (zero row
    first; zero-centred per (b, c) over T when asked), and the gradient of the
    scores = autograd through the fp64 restatement."""
    from torch_semimarkov_amd.streaming import emission_cum_scores

    g = torch.Generator().manual_seed(B * 1000 + T + C)
    x = (torch.randn(B, T, C, generator=g) + 0.3).to(dtype)
    x64 = x.double().requires_grad_(True)
    xs = x64 - x64.mean(dim=1, keepdim=True) if centre else x64
    want = torch.cat([torch.zeros(B, 1, C, dtype=torch.float64), xs.cumsum(1)], dim=1)
    xd = x.to(DEV).requires_grad_(True)
    got = emission_cum_scores(xd, zero_centre=centre)
    assert got.dtype == torch.float32 and got.shape == (B, T + 1, C)
    np.testing.assert_allclose(got.detach().cpu().double().numpy(), want.detach().numpy(), rtol=1e-7, atol=1e-6)
    gw = torch.randn(B, T + 1, C, generator=g)
    (gx,) = torch.autograd.grad((got * gw.to(DEV)).sum(), xd)
    (gx64,) = torch.autograd.grad((want * gw.double()).sum(), x64)
    assert gx.dtype == dtype
    tol = dict(rtol=1e-6, atol=1e-5) if dtype == torch.float32 else dict(rtol=1e-2, atol=1e-1)
    np.testing.assert_allclose(gx.cpu().double().numpy(), gx64.numpy(), **tol)


def test_emission_prologue_full_length_invariants():
    """T = 10^6, C = 24 (the headline shape): row 0 is zero, the last row is the
    column total (fp64 reference), centred columns end at ~0, and the head's
    cumulative scores are the prologue's."""
    from torch_semimarkov_amd.streaming import emission_cum_scores

    B, T, C = 1, 1_000_000, 24
    g = torch.Generator().manual_seed(77)
    x = torch.randn(B, T, C, generator=g)
    cum = emission_cum_scores(x.to(DEV)).cpu()
    assert torch.all(cum[:, 0] == 0)
    np.testing.assert_allclose(cum[:, -1].double().numpy(), x.double().sum(1).numpy(), rtol=1e-7, atol=1e-3)
    mid = x[:, :123457].double().sum(1)
    np.testing.assert_allclose(cum[:, 123457].double().numpy(), mid.numpy(), rtol=1e-7, atol=1e-3)
    cen = emission_cum_scores(x.to(DEV), zero_centre=True).cpu()
    assert cen[:, -1].abs().max() < 1e-3
    head = tsa.SemiMarkovCRFHead(C, 4).to(DEV)
    torch.testing.assert_close(head._cum_scores(x[:, :5000].to(DEV)), emission_cum_scores(x[:, :5000].to(DEV)),
                               rtol=0, atol=0)


# --------------------------------------------------------------------------- uncertainty consumers
def _oracle_uncertainty(head, hidden, L):
    """The reference's streaming uncertainty formulas (uncertainty.py:92-160, 263-368)
    evaluated with the fp64 oracle's backward."""
    with torch.no_grad():
        scores = head.projection(hidden) if head.projection is not None else hidden
    s = scores.detach().cpu().double().requires_grad_(True)
    B, T, C = s.shape
    cum = torch.cat([torch.zeros(B, 1, C, dtype=torch.float64), s.cumsum(1)], dim=1)
    tr = head.transition.detach().cpu().double()
    db = head.duration_bias.detach().cpu().double()
    part = R.streaming_oracle(cum, tr, db, L.cpu(), head.max_duration, "log")
    g_cum, g_s = torch.autograd.grad(part.sum(), (cum, s))
    boundary = g_cum[:, 1:].abs().sum(-1)
    pos = torch.softmax(g_s.abs(), dim=-1)
    p = boundary / (boundary.sum(-1, keepdim=True) + 1e-8)
    entropy = -(p * torch.log(p.clamp(min=1e-10))).sum(-1)
    return boundary, pos, entropy


@pytest.mark.parametrize("hidden_dim", [None, 16])
def test_uncertainty_consumers_vs_fp64_oracle(hidden_dim):
    B, T, C, K = 3, 80, 5, 9
    torch.manual_seed(11)
    head = tsa.UncertaintySemiMarkovCRFHead(C, K, hidden_dim=hidden_dim).to(DEV)
    g = torch.Generator().manual_seed(12)
    hidden = torch.randn(B, T, hidden_dim or C, generator=g).to(DEV)
    L = torch.tensor([80, 51, 7])
    want_b, want_p, want_h = _oracle_uncertainty(head, hidden, L)
    got_b = head.compute_boundary_marginals(hidden, L.to(DEV), normalize=False)
    np.testing.assert_allclose(got_b.cpu().double().numpy(), want_b.numpy(), rtol=1e-5, atol=1e-4)
    got_n = head.compute_boundary_marginals(hidden, L.to(DEV))
    want_n = want_b / (want_b.max(-1, keepdim=True)[0] + 1e-8)
    np.testing.assert_allclose(got_n.cpu().double().numpy(), want_n.numpy(), rtol=1e-5, atol=1e-5)
    got_p = head.compute_position_marginals(hidden, L.to(DEV))
    np.testing.assert_allclose(got_p.cpu().double().numpy(), want_p.numpy(), rtol=1e-5, atol=1e-5)
    got_h = head.compute_entropy_streaming(hidden, L.to(DEV))
    np.testing.assert_allclose(got_h.cpu().double().numpy(), want_h.numpy(), rtol=1e-5, atol=1e-5)
    labels = torch.randint(0, C, (B, T), generator=g).to(DEV)
    for mode in ("high_uncertainty", "boundary_regions"):
        lw = head.compute_loss_uncertainty_weighted(hidden, L.to(DEV), labels, 0.7, mode, reduction="none")
        nll = head.compute_loss(hidden, L.to(DEV), labels, reduction="none")
        u = got_h / (got_h.max() + 1e-8) if mode == "high_uncertainty" else got_n.mean(-1)
        torch.testing.assert_close(lw, nll * (1.0 + 0.7 * u), rtol=1e-5, atol=1e-5)
        lw.sum().backward()
    with pytest.raises(NotImplementedError):
        head.compute_boundary_marginals(hidden, L.to(DEV), use_streaming=False)
    with pytest.raises(NotImplementedError):
        head.compute_entropy_exact(hidden, L.to(DEV))


def test_uncertainty_marginals_are_probabilities():
    """Properties the forward-backward fixes: boundary signal at every interior
    position = 2 * P(boundary) summed over labels is in [0, 2]; position
    marginals sum to one."""
    B, T, C, K = 2, 500, 6, 20
    torch.manual_seed(3)
    head = tsa.UncertaintySemiMarkovCRFHead(C, K).to(DEV)
    hidden = torch.randn(B, T, C, device=DEV)
    L = torch.tensor([500, 320], device=DEV)
    sig = head.compute_boundary_marginals(hidden, L, normalize=False)
    assert sig.shape == (B, T) and bool((sig >= 0).all()) and bool((sig <= 2.0 + 1e-4).all())
    pm = head.compute_position_marginals(hidden, L)
    torch.testing.assert_close(pm.sum(-1), torch.ones(B, T, device=DEV), rtol=1e-5, atol=1e-5)


# --------------------------------------------------------------------------- gold-path score
GOLD_CASES = [(1, 3, 17, 4, 5), (2, 2, 9, 3, 1), (3, 4, 30, 5, 40), (4, 2, 1, 3, 4), (5, 3, 5000, 7, 300),
              (6, 2, 2100, 4, 3), (7, 3, 64, 130, 9)]


@pytest.mark.parametrize("seed,B,T,C,K", GOLD_CASES)
def test_score_gold_and_grads_vs_oracle(seed, B, T, C, K):
    """tsm_gold_score against the oracle's restatement of score_gold_vectorized
    (fp64), and its gradients against autograd through the oracle.  Long runs,
    runs longer than K-1, several position blocks (T = 5000) and K = 1 / T = 1."""
    g = torch.Generator().manual_seed(seed)
    cum = torch.zeros(B, T + 1, C)
    cum[:, 1:] = torch.randn(B, T, C, generator=g).cumsum(1)
    tr = torch.randn(C, C, generator=g)
    db = torch.randn(max(K, 2), C, generator=g)[:K] if K > 1 else torch.randn(2, C, generator=g)
    labels = torch.randint(0, C, (B, T), generator=g)
    labels[:, T // 3: T // 2] = 1  # long runs
    if T > 1000:
        labels[:, 1000:1700] = torch.randint(0, 2, (1,), generator=g).item()
    lengths = torch.randint(1, T + 1, (B,), generator=g)
    lengths[0] = T
    d = lambda x: x.double().requires_grad_(True)
    c64, t64, d64 = d(cum), d(tr), d(db)
    want = R.score_gold(c64, labels, lengths, t64, d64, K)
    gw = torch.linspace(0.5, 1.5, B, dtype=torch.float64)
    want_g = torch.autograd.grad((want * gw).sum(), (c64, t64, d64), allow_unused=True)
    want_g = [torch.zeros_like(x) if w is None else w for w, x in zip(want_g, (c64, t64, d64))]  # T == 1: no transition
    ins = [x.to(DEV).requires_grad_(True) for x in (cum, tr, db)]
    got = tsa.score_gold_vectorized(ins[0], labels.to(DEV), lengths.to(DEV), ins[1], ins[2], K)
    np.testing.assert_allclose(got.detach().cpu().double().numpy(), want.detach().numpy(), rtol=1e-6, atol=1e-4)
    got_g = torch.autograd.grad((got * gw.float().to(DEV)).sum(), ins)
    for a, w in zip(got_g, want_g):
        np.testing.assert_allclose(a.cpu().double().numpy(), w.numpy(), rtol=1e-6, atol=1e-6)


def test_score_gold_matches_reference_loss_fixture():
    z = load_golden("head_small")
    C, K = int(z["C"]), int(z["K"])
    hidden = torch.from_numpy(z["hidden"])
    cum = torch.zeros(hidden.shape[0], hidden.shape[1] + 1, C)
    cum[:, 1:] = torch.cumsum(hidden, 1)
    L = torch.from_numpy(z["lengths"])
    tr = torch.from_numpy(z["transition"])
    db = torch.from_numpy(z["duration_bias"])
    part, _, _ = R.forward(cum, tr, db, L, K)
    gold = tsa.score_gold_vectorized(cum.to(DEV), torch.from_numpy(z["labels"]).to(DEV), L.to(DEV), tr.to(DEV),
                                     db.to(DEV), K)
    np.testing.assert_allclose((part - gold.cpu()).numpy(), z["loss"], rtol=1e-5, atol=1e-4)


def test_score_gold_of_viterbi_path_is_viterbi_score():
    """Independent of the oracle: labelling the Viterbi segmentation (no two
    neighbouring segments share a label) and scoring it gives the Viterbi score
    minus the transition into the first segment (which the gold score omits)."""
    B, T, K, C = 3, 400, 12, 6
    cum, tr, db, L, _, _ = rand_problem(B, T, K, C, 6060, [400, 257, 3], tscale=0.5, dscale=0.5)
    tr = tr - 30.0 * torch.eye(C)
    score, cnt, segs = ops.viterbi(*to_dev(cum, tr, db, L), K, None, None, True, N.TSM_VITERBI_EXACT)
    labels = torch.zeros(B, T, dtype=torch.long)
    first_tr = torch.zeros(B)
    segs = segs.cpu()
    for b in range(B):
        for i in range(int(cnt[b])):
            s, e, c, cp = (int(v) for v in segs[b, i])
            labels[b, s:e + 1] = c
            if s == 0:
                first_tr[b] = tr[cp, c]
    gold = tsa.score_gold_vectorized(*to_dev(cum, labels, L, tr, db), K).cpu()
    np.testing.assert_allclose(gold.double().numpy(), (score.cpu() - first_tr).double().numpy(), rtol=2e-6)


def test_score_gold_flags_out_of_range_labels():
    cum = torch.randn(2, 11, 3).cumsum(1).to(DEV)
    labels = torch.zeros(2, 10, dtype=torch.long)
    labels[1, 4] = 7  # outside [0, C) inside the sequence
    labels[0, 9] = 9  # outside the sequence (length 8): ignored
    L = torch.tensor([8, 10])
    got = tsa.score_gold_vectorized(cum, labels.to(DEV), L.to(DEV), torch.zeros(3, 3, device=DEV),
                                    torch.zeros(4, 3, device=DEV), 4).cpu()
    assert torch.isfinite(got[0]) and torch.isnan(got[1])


# --------------------------------------------------------------------------- head
@pytest.mark.parametrize("name", ["head_small", "head_proj"])
def test_head_matches_reference_golden(name):
    z = load_golden(name)
    C, K = int(z["C"]), int(z["K"])
    H = z["hidden"].shape[-1]
    head = tsa.SemiMarkovCRFHead(C, K, hidden_dim=H if "proj_weight" in z else None).to(DEV)
    with torch.no_grad():
        head.transition.copy_(torch.from_numpy(z["transition"]))
        head.duration_dist.duration_bias.copy_(torch.from_numpy(z["duration_bias"]))
        if head.projection is not None:
            head.projection.weight.copy_(torch.from_numpy(z["proj_weight"]))
            head.projection.bias.copy_(torch.from_numpy(z["proj_bias"]))
    hidden = torch.from_numpy(z["hidden"]).to(DEV)
    L = torch.from_numpy(z["lengths"]).to(DEV)
    labels = torch.from_numpy(z["labels"]).to(DEV)
    loss = head.compute_loss(hidden, L, labels, reduction="none")
    np.testing.assert_allclose(loss.detach().cpu().numpy(), z["loss"], rtol=1e-5, atol=1e-4)
    loss.sum().backward()
    np.testing.assert_allclose(head.transition.grad.cpu().numpy(), z["grad_transition"], **GRAD_TOL)
    np.testing.assert_allclose(head.duration_dist.duration_bias.grad.cpu().numpy(), z["grad_duration_bias"],
                               **GRAD_TOL)
    if head.projection is not None:
        np.testing.assert_allclose(head.projection.weight.grad.cpu().numpy(), z["grad_proj_weight"],
                                   rtol=1e-5, atol=2e-4)
    with torch.no_grad():
        part = head(hidden, L)["partition"]
        vit = head.decode(hidden, L)
        res = head.decode_with_traceback(hidden, L, int(z["max_traceback_length"]))
    np.testing.assert_allclose(part.cpu().numpy(), z["partition"], rtol=1e-5, atol=1e-5)
    # the head builds cum_scores with the GPU's cumsum/Linear, whose fp32 rounding differs
    # from the reference's CPU run, so head-level scores agree to 1e-5 (the scan itself is
    # bit-exact for identical cum_scores, see test_inference_matches_reference_golden)
    np.testing.assert_allclose(vit.cpu().numpy(), z["viterbi"], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(res.scores.cpu().numpy(), z["traceback_scores"], rtol=1e-5, atol=1e-5)
    assert torch.equal(res.scores, vit)
    got = [(b, s.start, s.end, s.label) for b, sl in enumerate(res.segments) for s in sl]
    np.testing.assert_array_equal(np.array(got, dtype=np.int64).reshape(-1, 4), z["segments"])
    sc = np.array([s.score for sl in res.segments for s in sl])
    np.testing.assert_allclose(sc, z["segment_scores"], rtol=1e-5, atol=1e-5)
    for b, sl in enumerate(res.segments):
        assert abs(sum(s.score for s in sl) - res.scores[b].item()) < 1e-4


def test_traceback_skips_long_sequences():
    head = tsa.SemiMarkovCRFHead(3, 5).to(DEV)
    hidden = torch.randn(2, 30, 3, device=DEV)
    res = head.decode_with_traceback(hidden, torch.tensor([30, 12], device=DEV), max_traceback_length=20)
    assert res.segments[0] == [] and len(res.segments[1]) >= 1
    assert res.segments[1][0].start == 0 and res.segments[1][-1].end == 11


def test_segment_terms_match_host_gathers():
    """tsm_segment_terms against the same terms gathered on the host from the traceback
    rows: content as the fp32 difference of two cum entries, duration bias at
    min(end-start+1, K-1), transition from the previous label (ragged lengths, a
    length-1 sequence); the segment scores sum to the Viterbi score."""
    B, T, K, C = 4, 300, 12, 6
    cum, tr, db, L, _, _ = rand_problem(B, T, K, C, 515, [300, 1, 173, 299])
    cum_d, tr_d, db_d, L_d = cum.to(DEV), tr.to(DEV), db.to(DEV), L.to(DEV)
    score, cnt, segs = ops.viterbi(cum_d, tr_d, db_d, L_d, K, None, None, True)
    out = ops.segment_terms(cum_d, tr_d, db_d, cnt, segs, K).cpu().numpy()
    cnt, segs = cnt.cpu().numpy(), segs.cpu().numpy()
    cum_n, tr_n, db_n = cum.numpy(), tr.numpy(), db.numpy()
    for b in range(B):
        n = int(cnt[b])
        assert n >= 1
        s, e, lab, pv = (segs[b, :n, i].astype(np.int64) for i in range(4))
        content = (cum_n[b, e + 1, lab] - cum_n[b, s, lab]).astype(np.float64)  # fp32 difference
        want = np.stack([s, e, lab, content, db_n[np.minimum(e - s + 1, K - 1), lab].astype(np.float64),
                         tr_n[pv, lab].astype(np.float64)], axis=-1)
        np.testing.assert_array_equal(out[b, :n], want)
        total = ((out[b, :n, 3] + out[b, :n, 4]) + out[b, :n, 5]).sum()
        assert abs(total - score[b].item()) <= 1e-5 * max(1.0, abs(total)) + 1e-4


# --------------------------------------------------------------------------- launcher contracts
def test_launcher_checkpoints_and_backward_contract():
    z = load_golden("stream_varlen")
    cum, tr, db, L, K, sr, ps, pe = fixture_inputs(z)
    part, ck, S = launch_streaming_hip_kernel(cum, tr, db, L, K)
    assert S == int(z["checkpoint_interval"])
    want = torch.from_numpy(z["ring_checkpoints"])
    assert ck.shape == want.shape
    np.testing.assert_allclose(ck.cpu().numpy(), want.numpy(), rtol=1e-5, atol=1e-4)
    g = torch.ones(cum.shape[0], device=DEV)
    gc, gt, gd, gps, gpe = launch_streaming_hip_backward(cum, tr, db, L, part, ck, S, g)
    assert gps is None and gpe is None
    assert_grads([gc.cpu(), gt.cpu(), gd.cpu()],
                 [torch.from_numpy(z[k]) for k in ("grad_cum", "grad_transition", "grad_duration_bias")])


@pytest.mark.parametrize("marginals", ["default", "separate"])
def test_kernel_timing_counts_launches(marginals, monkeypatch):
    if marginals == "separate":
        monkeypatch.setenv("TSM_MARGINAL_PATH", "separate")
    else:
        monkeypatch.delenv("TSM_MARGINAL_PATH", raising=False)
    z = load_golden("stream_medium")
    cum, tr, db, L, K, sr, ps, pe = fixture_inputs(z, requires_grad=True)
    B, Tp1, C = cum.shape
    fused = N.plan_info(B, Tp1 - 1, C, K)["mfused"] == 1
    assert fused == (marginals == "default"), marginals
    N.timing_enable(True)
    try:
        part = tsa.semi_crf_streaming_forward(cum, tr, db, L, K, semiring=sr)
        part.sum().backward()
        torch.cuda.synchronize()
        t = N.timing_read()
    finally:
        N.timing_enable(False)
    rows = ("u_rows_kernel", "fused_rows_kernel") if fused else ("marginal_kernel", "finalize_rows_kernel")
    for name in ("scan_fwd_kernel", "scan_bwd_kernel") + rows:
        ms, n = t[name]
        assert n == 1 and ms > 0.0, (name, t[name])
    # disabled: nothing more is recorded
    part = tsa.semi_crf_streaming_forward(cum.detach(), tr.detach(), db.detach(), L, K, semiring=sr)
    torch.cuda.synchronize()
    assert N.timing_read() == {}

