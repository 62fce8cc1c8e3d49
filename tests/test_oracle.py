"""Pins the CPU oracle (oracle/streaming_ref.py) -- CPU only.

Each check is independent of the oracle's own recursion: exhaustive
enumeration, a probability-space HMM, the reference's T=1 known answer,
finite differences, exact identities of the marginals, and golden vectors
produced by the reference itself (tests/golden/make_golden.py).
"""

import numpy as np
import pytest
import torch

from conftest import load_golden
from oracle import brute as BR
from oracle import streaming_ref as R

STREAM_FIXTURES = [
    "stream_basic", "stream_varlen", "stream_k1", "stream_c24", "stream_t1", "stream_t2",
    "stream_proj", "stream_durtrans", "stream_max", "stream_nocentre", "stream_medium",
]


def rand_problem(B, T, K, C, seed, dtype=torch.float64, lengths=None, dur_trans=False):
    g = torch.Generator().manual_seed(seed)
    cum = torch.zeros(B, T + 1, C, dtype=dtype)
    cum[:, 1:] = torch.randn(B, T, C, generator=g, dtype=dtype).cumsum(1)
    tr = 0.3 * torch.randn(*((K, C, C) if dur_trans else (C, C)), generator=g, dtype=dtype)
    db = 0.3 * torch.randn(K, C, generator=g, dtype=dtype)
    if lengths is None:
        lengths = torch.full((B,), T, dtype=torch.long)
    else:
        lengths = torch.tensor(lengths, dtype=torch.long)
    ps = 0.2 * torch.randn(B, T, C, generator=g, dtype=dtype)
    pe = 0.2 * torch.randn(B, T, C, generator=g, dtype=dtype)
    return cum, tr, db, lengths, ps, pe


# --------------------------------------------------------------------------- brute force
@pytest.mark.parametrize("B,T,K,C,lengths", [
    (2, 6, 4, 3, [6, 4]), (1, 5, 1, 3, None), (2, 7, 3, 2, [7, 5]), (1, 1, 5, 2, None),
    (1, 8, 9, 2, None), (3, 5, 2, 2, [5, 3, 1]),
])
@pytest.mark.parametrize("semiring", ["log", "max"])
@pytest.mark.parametrize("proj", [False, True])
def test_forward_matches_enumeration(B, T, K, C, lengths, semiring, proj):
    cum, tr, db, L, ps, pe = rand_problem(B, T, K, C, 7 + T + K, lengths=lengths)
    a, b = (ps, pe) if proj else (None, None)
    got, _, _ = R.forward(cum, tr, db, L, K, semiring, a, b)
    want = BR.brute_log_partition(cum, tr, db, L, K, semiring, a, b)
    torch.testing.assert_close(got, want, rtol=0, atol=1e-12)


@pytest.mark.parametrize("B,T,K,C,lengths,dur_trans", [
    (2, 6, 4, 3, [6, 4], False), (1, 5, 1, 3, None, False), (2, 7, 3, 2, [7, 5], False),
    (2, 6, 4, 2, [6, 5], True),
])
@pytest.mark.parametrize("proj", [False, True])
def test_gradients_match_enumeration(B, T, K, C, lengths, dur_trans, proj):
    cum, tr, db, L, ps, pe = rand_problem(B, T, K, C, 11 + T, lengths=lengths, dur_trans=dur_trans)
    ins = [cum, tr, db] + ([ps, pe] if proj else [])
    for x in ins:
        x.requires_grad_(True)
    g = torch.linspace(0.5, 2.0, B, dtype=torch.float64)
    a, b = (ps, pe) if proj else (None, None)
    got = torch.autograd.grad((R.streaming_oracle(cum, tr, db, L, K, "log", a, b) * g).sum(), ins)
    want = torch.autograd.grad((BR.brute_log_partition(cum, tr, db, L, K, "log", a, b) * g).sum(), ins)
    for x, y in zip(got, want):
        torch.testing.assert_close(x, y, rtol=0, atol=1e-11)


def test_max_soft_marginals_match_enumeration():
    """Max-semiring backward ("soft max-marginals", pytorch_reference.py:458-467,513-518).

    alpha[s,c'] / beta[s,c'] are taken as the best prefix / suffix score over all
    enumerated full paths with a boundary at s whose segment ending at s has
    label c' (the virtual start label for s=0); the expected duration gradient
    is sum over segments of exp(alpha + edge + beta - best).
    """
    B, T, K, C = 1, 6, 4, 2
    cum, tr, db, L, _, _ = rand_problem(B, T, K, C, 5)
    part, ck, S = R.forward(cum, tr, db, L, K, "max")
    res = R.backward(cum, tr, db, L, K, part, ck, S, "max")

    def seg_val(s, k, c):
        return float(cum[0, s + k, c] - cum[0, s, c] + db[min(k, K - 1), c])

    alpha, beta = {}, {}
    best = -1e30
    for c0, segs in BR.enumerate_paths(T, K, C):
        labels = [c0] + [c for (_, _, c) in segs]
        pieces = [seg_val(s, k, c) + float(tr[labels[i], c]) for i, (s, k, c) in enumerate(segs)]
        total = sum(pieces)
        best = max(best, total)
        run = 0.0
        for i, (s, k, c) in enumerate(segs):
            key = (s, labels[i])
            alpha[key] = max(alpha.get(key, -1e30), run)
            beta[key] = max(beta.get(key, -1e30), total - run)
            run += pieces[i]
        beta[(T, labels[-1])] = 0.0
    g_db = torch.zeros(K, C, dtype=torch.float64)
    for s in range(T):
        for k in BR.allowed_durations(K):
            if s + k > T:
                continue
            for c in range(C):
                for cp in range(C):
                    if (s, cp) in alpha and (s + k, c) in beta:
                        e = seg_val(s, k, c) + float(tr[cp, c])
                        g_db[min(k, K - 1), c] += np.exp(alpha[(s, cp)] + e + beta[(s + k, c)] - best)
    assert abs(float(part[0]) - best) < 1e-12
    torch.testing.assert_close(res.grad_duration_bias[0], g_db, rtol=1e-10, atol=1e-12)


def test_gradcheck_fp64():
    """Finite differences, as tests/test_streaming.py:229-251 does for the reference."""
    cum, tr, db, L, ps, pe = rand_problem(1, 10, 4, 2, 3)
    for x in (cum, tr, db, ps, pe):
        x.requires_grad_(True)
    torch.autograd.gradcheck(
        lambda a, b, c, d, e: R.streaming_oracle(a, b, c, L, 4, "log", d, e),
        (cum, tr, db, ps, pe), eps=1e-6, atol=1e-6, rtol=1e-5,
    )


# --------------------------------------------------------------------------- closed forms
def test_t1_known_answer():
    """tests/test_edge_cases.py:167-193: C=2, content (2,1), db[1]=1, trans 0."""
    cum = torch.zeros(1, 2, 2)
    cum[0, 1] = torch.tensor([2.0, 1.0])
    tr = torch.zeros(2, 2)
    db = torch.zeros(5, 2)
    db[1] = 1.0
    got, _, _ = R.forward(cum, tr, db, torch.tensor([1]), 5)
    log2 = float(np.log(2.0))
    want = torch.logsumexp(torch.tensor([2 + 1 + log2, 1 + 1 + log2]), 0)
    torch.testing.assert_close(got[0], want, rtol=0, atol=1e-6)
    torch.testing.assert_close(got[0], BR.t1_closed_form(cum[0], tr, db), rtol=0, atol=1e-6)


def test_k1_equals_probability_space_hmm():
    T, C = 300, 5
    cum, tr, db, L, _, _ = rand_problem(1, T, 1, C, 21)
    cum.requires_grad_(True)
    tr.requires_grad_(True)
    part = R.streaming_oracle(cum, tr, db, L, 1)
    gc, gt = torch.autograd.grad(part.sum(), [cum, tr])
    logZ, state_post, trans_counts, _ = BR.hmm_forward_backward(
        cum[0].detach().numpy(), tr.detach().numpy(), db[0].numpy(), T
    )
    assert abs(part.item() - logZ) < 1e-9 * abs(logZ)
    # d logZ / d cum[t, c] = P(label t-1 = c) - P(label t = c)
    want = np.zeros((T + 1, C))
    want[1:] += state_post
    want[:-1] -= state_post
    np.testing.assert_allclose(gc[0].numpy(), want, atol=1e-10)
    np.testing.assert_allclose(gt.numpy(), trans_counts, atol=1e-9)


def test_gradient_identities():
    """Exact consequences of the backward: rows of grad_cum sum to 0 over t; the
    final row sums to +1 and row 0 to -1 over labels; sum(grad_trans) = sum(grad_db)."""
    cum, tr, db, L, _, _ = rand_problem(2, 40, 6, 4, 31, lengths=[40, 27])
    for x in (cum, tr, db):
        x.requires_grad_(True)
    g = torch.tensor([1.0, 1.0], dtype=torch.float64)
    res_part, ck, S = R.forward(cum.detach(), tr.detach(), db.detach(), L, 6)
    res = R.backward(cum.detach(), tr.detach(), db.detach(), L, 6, res_part, ck, S)
    for b, Lb in enumerate([40, 27]):
        gc = res.grad_cum[b]
        np.testing.assert_allclose(gc.sum(0).numpy(), 0.0, atol=1e-12)
        assert abs(gc[Lb].sum().item() - 1.0) < 1e-12
        assert abs(gc[0].sum().item() + 1.0) < 1e-12
        assert abs(res.grad_transition[b].sum().item() - res.grad_duration_bias[b].sum().item()) < 1e-10
        assert torch.all(gc[Lb + 1:] == 0)


def test_checkpoint_interval_rule():
    """pytorch_reference.py:25-45 and tests/test_edge_cases_extended.py:533-567."""
    assert R.checkpoint_interval(1000, 100) == 316
    assert R.checkpoint_interval(10_000, 1) == 100
    assert R.checkpoint_interval(1_000_000, 300) == 17320
    assert R.checkpoint_interval(8192, 64) == 724
    assert R.checkpoint_interval(50_000, 500) == 5000
    assert R.checkpoint_interval(10, 100) == 100  # clamped to >= K


# --------------------------------------------------------------------------- golden vectors
@pytest.mark.parametrize("name", STREAM_FIXTURES)
def test_oracle_fp32_matches_reference_golden(name):
    z = load_golden(name)
    cum = torch.from_numpy(z["cum"])
    tr = torch.from_numpy(z["transition"])
    db = torch.from_numpy(z["duration_bias"])
    L = torch.from_numpy(z["lengths"])
    K = int(z["K"])
    sr = str(z["semiring"])
    ps = torch.from_numpy(z["proj_start"]) if "proj_start" in z else None
    pe = torch.from_numpy(z["proj_end"]) if "proj_end" in z else None
    part, ck, S = R.forward(cum, tr, db, L, K, sr, ps, pe)
    # forward: the same stacked tensors go into the same reductions -> bit-identical
    assert torch.equal(part, torch.from_numpy(z["partition_raw"]))
    assert torch.equal(ck, torch.from_numpy(z["ring_checkpoints"]))
    assert S == int(z["checkpoint_interval"])
    res = R.backward(cum, tr, db, L, K, part, ck, S, sr, ps, pe)
    g = torch.from_numpy(z["grad_output"])
    gc, gt, gd, gps, gpe = R.scale_backward(res, g)
    tol = dict(rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(gc.numpy(), z["grad_cum"], **tol)
    np.testing.assert_allclose(gt.numpy(), z["grad_transition"], **tol)
    np.testing.assert_allclose(gd.numpy(), z["grad_duration_bias"], **tol)
    if ps is not None:
        np.testing.assert_allclose(gps.numpy(), z["grad_proj_start"], **tol)
        np.testing.assert_allclose(gpe.numpy(), z["grad_proj_end"], **tol)


@pytest.mark.parametrize("name", ["head_small", "head_proj"])
def test_oracle_traceback_matches_reference_golden(name):
    z = load_golden(name)
    C, K = int(z["C"]), int(z["K"])
    hidden = torch.from_numpy(z["hidden"])
    if "proj_weight" in z:
        scores = hidden @ torch.from_numpy(z["proj_weight"]).T + torch.from_numpy(z["proj_bias"])
    else:
        scores = hidden
    B, T, _ = scores.shape
    cum = torch.zeros(B, T + 1, C)
    cum[:, 1:] = torch.cumsum(scores.float(), dim=1)
    tr = torch.from_numpy(z["transition"])
    db = torch.from_numpy(z["duration_bias"])
    L = torch.from_numpy(z["lengths"])
    seg_ref = z["segments"]
    sc_ref = z["segment_scores"]
    part_max, _, _ = R.forward(cum, tr, db, L, K, "max")
    np.testing.assert_allclose(part_max.numpy(), z["traceback_scores"], rtol=1e-6, atol=1e-5)
    got = []
    got_sc = []
    for b in range(B):
        segs, best = R.viterbi_traceback_single(cum[b], tr, db, K, int(L[b]))
        assert best == float(part_max[b])  # same fp32 max table
        for (s, e, l, cp) in segs:
            got.append((b, s, e, l))
            got_sc.append(R.segment_score(cum[b], tr, db, K, s, e, l, cp))
    np.testing.assert_array_equal(np.array(got).reshape(-1, 4), seg_ref)
    np.testing.assert_allclose(np.array(got_sc), sc_ref, rtol=1e-6, atol=1e-5)
    # gold score of the labels (helpers.py:365-544) -> loss = partition - gold
    part_log, _, _ = R.forward(cum, tr, db, L, K, "log")
    gold = R.score_gold(cum, torch.from_numpy(z["labels"]), L, tr, db, K)
    np.testing.assert_allclose((part_log - gold).numpy(), z["loss"], rtol=1e-5, atol=1e-4)


# --------------------------------------------------------------------------- the C restatement (oracle/cref.py)
CREF_CASES = [
    (2, 30, 5, 4, None, False), (3, 40, 6, 3, [40, 17, 0], True), (2, 20, 1, 3, [20, 9], False),
    (1, 60, 8, 24, None, False), (2, 25, 30, 5, [25, 3], True), (1, 1, 4, 3, None, True),
]


@pytest.mark.parametrize("B,T,K,C,lengths,proj", CREF_CASES)
def test_cref_forward_backward_match_streaming_ref(B, T, K, C, lengths, proj):
    """The label-factorised C restatement against the direct K*C^2 recursion of
    oracle/streaming_ref.py (fp64): partition in both semirings and every
    gradient, with projections, ragged and zero lengths, K=1 and T=1."""
    from oracle import cref

    cum, tr, db, L, ps, pe = rand_problem(B, T, K, C, 101 + T + K, lengths=lengths)
    a, b = (ps, pe) if proj else (None, None)
    for sr in ("log", "max"):
        got = cref.forward(cum, tr, db, L, K, sr, a, b)
        want, _, _ = R.forward(cum, tr, db, L, K, sr, a, b)
        np.testing.assert_allclose(got, want.numpy(), rtol=1e-12, atol=1e-9)
    res = cref.backward(cum, tr, db, L, K, a, b)
    part, ck, S = R.forward(cum, tr, db, L, K, "log", a, b)
    br = R.backward(cum, tr, db, L, K, part, ck, S, "log", a, b)
    pairs = [("grad_cum", br.grad_cum), ("grad_transition", br.grad_transition),
             ("grad_duration_bias", br.grad_duration_bias)]
    if proj:
        pairs += [("grad_proj_start", br.grad_proj_start), ("grad_proj_end", br.grad_proj_end)]
    for key, want in pairs:
        np.testing.assert_allclose(res[key], want.numpy(), rtol=1e-10, atol=1e-11, err_msg=key)


def test_cref_backward_matches_enumeration_and_identities():
    """Exact marginals by enumeration (tiny problem) and the identities on a
    medium one: every segment has one start, one end, one duration and one
    incoming transition."""
    from oracle import cref

    cum, tr, db, L, ps, pe = rand_problem(2, 6, 4, 3, 5, lengths=[6, 4])
    ins = [x.clone().requires_grad_(True) for x in (cum, tr, db)]
    z = BR.brute_log_partition(ins[0], ins[1], ins[2], L, 4, "log")
    want = torch.autograd.grad(z.sum(), ins)
    res = cref.backward(cum, tr, db, L, 4)
    np.testing.assert_allclose(res["grad_cum"], want[0].numpy(), atol=1e-12)
    np.testing.assert_allclose(res["grad_transition"].sum(0), want[1].numpy(), atol=1e-12)
    np.testing.assert_allclose(res["grad_duration_bias"].sum(0), want[2].numpy(), atol=1e-12)
    cum, tr, db, L, _, _ = rand_problem(2, 700, 40, 7, 6, lengths=[700, 333])
    res = cref.backward(cum, tr, db, L, 40)
    gc = res["grad_cum"]
    for b in range(2):
        n = int(L[b])
        np.testing.assert_allclose(gc[b].sum(0), 0.0, atol=1e-9)
        assert abs(gc[b, n].sum() - 1) < 1e-10 and abs(gc[b, 0].sum() + 1) < 1e-10
        assert np.all(gc[b, n + 1:] == 0)
        n_seg = res["grad_duration_bias"][b].sum()
        assert abs(res["grad_transition"][b].sum() - n_seg) < 1e-9 * n_seg


@pytest.mark.parametrize("B,T,K,C,lengths", [(2, 30, 5, 4, None), (2, 20, 1, 3, [20, 9]), (1, 60, 8, 24, None),
                                             (3, 45, 12, 5, [45, 0, 7])])
def test_cref_viterbi_matches_traceback_restatement(B, T, K, C, lengths):
    """The C Viterbi against ``viterbi_traceback_single`` (itself pinned by the
    reference's fixtures and by brute force): fp32 tables bit-identical
    (scores and segments), fp64 segments and scores equal."""
    from oracle import cref

    cum, tr, db, L, _, _ = rand_problem(B, T, K, C, 211 + C, lengths=lengths)
    for dt, tdt in ((np.float32, torch.float32), (np.float64, torch.float64)):
        v = cref.viterbi(cum, tr, db, L, K, dtype=dt)
        for b in range(B):
            n = int(L[b])
            if n == 0:
                assert v["segments"][b] == []
                continue
            segs, sc = R.viterbi_traceback_single(cum[b].to(tdt), tr.to(tdt), db.to(tdt), K, n)
            assert v["segments"][b] == [tuple(s) for s in segs], (dt, b)
            assert v["score"][b] == sc, (dt, b)


def test_cref_viterbi_gaps_and_exact_ties():
    """The tie bookkeeping of the fp64 Viterbi.  (1) min_gap equals the
    smallest nonzero best-minus-runner-up gap over the backtrace's decisions,
    recomputed here from the restatement's fp64 alpha table.  (2) A run of one
    label cut into two segments of different durations has an exact twin (the
    durations swapped): it is counted as a tie, not as a small gap."""
    from oracle import cref

    cum, tr, db, L, _, _ = rand_problem(1, 40, 6, 3, 17)
    v = cref.viterbi(cum, tr, db, L, 6, dtype=np.float64, close_thr=0.5)
    _, _, _, alpha = R.forward(cum, tr, db, L, 6, "max", return_alpha=True)
    alpha = alpha[0].numpy()
    c64, t64, d64 = cum[0].numpy(), tr.numpy(), db.numpy()
    gaps = []
    fin = np.sort(alpha[40])[::-1]
    gaps.append(fin[0] - fin[fin < fin[0]].max())
    for (s, e, c, cp) in v["segments"][0]:
        t = e + 1
        cands = [alpha[t - k, q] + ((c64[t, c] - c64[t - k, c]) + d64[min(k, 5), c]) + t64[q, c]
                 for k in range(1, min(5, t) + 1) for q in range(3)]
        cands = np.sort(np.array(cands))[::-1]
        lower = cands[cands < cands[0]]
        if lower.size:
            gaps.append(cands[0] - lower[0])
    assert abs(v["min_gap"][0] - min(gaps)) < 1e-12
    assert v["n_close"][0] == sum(g < 0.5 for g in gaps)
    # exact twin: label 0 is the only good label and a self-transition bonus
    # makes two segments (durations 2 and 3) beat one of duration 5
    T, K, C = 5, 6, 2
    cum = torch.zeros(1, T + 1, C, dtype=torch.float64)
    cum[0, 1:, 0] = torch.arange(1, T + 1, dtype=torch.float64)
    cum[0, 1:, 1] = -10.0 * torch.arange(1, T + 1, dtype=torch.float64)
    tr = torch.tensor([[1.0, -5.0], [-5.0, -5.0]], dtype=torch.float64)
    db = torch.zeros(K, C, dtype=torch.float64)
    db[1] = db[4] = db[5] = -3.0
    v = cref.viterbi(cum.float(), tr.float(), db.float(), torch.tensor([T]), K, dtype=np.float64)
    durs = sorted(e - s + 1 for (s, e, c, cp) in v["segments"][0])
    assert durs == [2, 3] and v["n_ties"][0] >= 1
