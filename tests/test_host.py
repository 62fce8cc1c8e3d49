"""Host-side checks that need no GPU: the C ABI library loads and exports every
declared symbol, plans/workspaces and error paths behave, the Python layer
validates inputs and fails loudly off-GPU, and the device-agnostic helpers
match the oracle."""

import ctypes
import os
import re

import numpy as np
import pytest
import torch

from conftest import ROOT, load_golden
from oracle import streaming_ref as R

import torch_semimarkov_amd as tsa
from torch_semimarkov_amd import _native as N
from torch_semimarkov_amd.streaming import compute_edge_block_streaming

HEADER = os.path.join(ROOT, "include", "tsm_hip.h")


def declared_symbols():
    txt = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(tsm_\w+)\(", txt, re.M)))


def test_library_exports_every_declared_symbol():
    lib = N.lib()
    decl = declared_symbols()
    assert len(decl) >= 10
    for name in decl:
        assert hasattr(lib, name), name
    assert sorted(N.EXPORTED) == decl


def test_version_and_error_message():
    lib = N.lib()
    assert lib.tsm_version() >= 100
    out = ctypes.c_size_t(0)
    rc = lib.tsm_forward_workspace(0, 10, 4, 3, 0, 0, 0, 0, ctypes.byref(out))
    assert rc == 1
    assert b"B, T, C, K" in lib.tsm_last_error()
    rc = lib.tsm_forward_workspace(1, 10, 4, 3, 0, 7, 0, 0, ctypes.byref(out))
    assert rc == 1 and b"semiring" in lib.tsm_last_error()


def test_plan_and_workspace_queries_without_gpu():
    p = N.plan_info(1, 1_000_000, 24, 300)
    assert p["Kmax"] == 299 and p["J"] == 16 and p["NT"] == 384
    assert p["RS"] >= p["Kmax"] + 2 and p["RS"] % 32 == 16
    assert p["P"] > 1 and p["Lc"] * p["P"] >= 1_000_000 and p["Lc"] >= 4 * p["W"]
    assert p["TB"] >= p["Kmax"] and p["NB"] * p["TB"] >= 1_000_000
    # few short sequences leave most CUs idle: chunks of about one warm-up each
    s = N.plan_info(4, 1000, 24, 100)
    assert s["P"] == 1000 // s["W"] and s["Lc"] >= s["W"], s
    # a sequence shorter than two warm-ups runs in one chunk
    assert N.plan_info(4, 300, 24, 100)["P"] == 1
    # large label spaces split the marginal kernel into label blocks
    q = N.plan_info(8, 50_000, 128, 500)
    assert q["CB"] * q["NCB"] >= 128 and q["marg_lds"] <= 160 * 1024
    for tr_rows in (0, 5):
        for fn, args in (
            (N.lib().tsm_forward_workspace, (2, 100, 8, 5, tr_rows, 0, 0, 0)),
            (N.lib().tsm_backward_workspace, (2, 100, 8, 5, tr_rows, 1, 1)),
            (N.lib().tsm_viterbi_workspace, (2, 100, 8, 5, tr_rows, 1)),
        ):
            out = ctypes.c_size_t(0)
            assert fn(*args, ctypes.byref(out)) == 0 and out.value > 0


def test_duration_dependent_transition_plans_without_gpu():
    """(K, C, C) transitions: the dense path replaces the factorised ones; one
    matrix per duration index 1..max(K-1, 1) is required; C <= 128."""
    p = N.plan_info(2, 3000, 8, 12, trans_rows=12)
    assert p["dense"] == 1 and p["fast"] == 0 and p["mfast"] == 0
    assert p["DNT"] % 64 == 0 and p["DNT"] >= 8 * p["DJ"] and p["dtrl"] == 1
    assert p["DTB"] >= p["Kmax"] and p["DNB"] * p["DTB"] >= 3000
    assert p["DG"] >= 8 and p["DNTM"] <= 1024
    # transitions too large for LDS are read from the global table
    big = N.plan_info(1, 1000, 64, 100, trans_rows=100)
    assert big["dense"] == 1 and big["dtrl"] == 0
    assert N.plan_info(2, 100, 8, 5)["dense"] == 0
    lib = N.lib()
    out = (ctypes.c_int64 * 4)()
    assert lib.tsm_plan_info(2, 100, 8, 5, 4, 0, 0, out, 4) == 1  # needs >= Kmax + 1 = 5 matrices
    assert b"trans_rows >= 5" in lib.tsm_last_error()
    assert lib.tsm_plan_info(2, 100, 8, 1, 1, 0, 0, out, 4) == 1  # K = 1 uses duration 1: two matrices
    assert lib.tsm_plan_info(2, 100, 8, 1, 2, 0, 0, out, 4) == 0
    assert lib.tsm_plan_info(2, 100, 200, 5, 5, 0, 0, out, 4) == 2
    assert lib.tsm_plan_info(2, 100, 8, 5, -1, 0, 0, out, 4) == 1


def test_c_abi_rejects_bad_calls_without_touching_the_device():
    lib = N.lib()
    # missing required pointers
    rc = lib.tsm_forward(None, None, None, None, None, None, 1, 10, 4, 3, 0, 0, None, None, None, None, None,
                         None, 0, None)
    assert rc == 1
    # workspace too small is reported before any launch
    buf = ctypes.create_string_buffer(16)
    fake = ctypes.addressof(buf)
    rc = lib.tsm_forward(fake, fake, fake, fake, None, None, 1, 10, 4, 3, 0, 0, fake, None, None, None, None,
                         fake, 1, None)
    assert rc == 4 and b"workspace" in lib.tsm_last_error()
    rc = lib.tsm_forward(fake, fake, fake, fake, None, None, 1, 10, 4, 3, 0, 0, fake, None, fake, None, None,
                         fake, 10**9, None)
    assert rc == 1 and b"alpha_hat and alpha_level" in lib.tsm_last_error()
    rc = lib.tsm_plan_info(1, 10, 600, 3, 0, 0, 0, None, 0)
    assert rc == 2
    # segment terms: required pointers and sizes are checked before any launch
    rc = lib.tsm_segment_terms(fake, fake, fake, None, fake, 1, 10, 4, 3, fake, None)
    assert rc == 1 and b"seg_count" in lib.tsm_last_error()
    rc = lib.tsm_segment_terms(fake, fake, fake, fake, fake, 1, 10, 0, 3, fake, None)
    assert rc == 1 and b"C, K >= 1" in lib.tsm_last_error()


def test_python_api_fails_loudly_off_gpu():
    cum = torch.zeros(1, 6, 3)
    tr = torch.zeros(3, 3)
    db = torch.zeros(4, 3)
    L = torch.tensor([5])
    with pytest.raises(ValueError, match="semiring"):
        tsa.semi_crf_streaming_forward(cum, tr, db, L, 4, semiring="sum")
    with pytest.raises(RuntimeError, match="AMD GPU"):
        tsa.semi_crf_streaming_forward(cum, tr, db, L, 4)
    head = tsa.SemiMarkovCRFHead(3, 4)
    with pytest.raises(RuntimeError, match="AMD GPU"):
        head(torch.zeros(1, 5, 3), L)


def test_reference_head_initialisation_order():
    """Seeded init draws transition, then duration bias, then the projection (nn.py:146-162)."""
    z = load_golden("head_proj")
    torch.manual_seed(202)
    head = tsa.SemiMarkovCRFHead(num_classes=6, max_duration=12, hidden_dim=16)
    np.testing.assert_array_equal(head.transition.detach().numpy(), z["transition"])
    np.testing.assert_array_equal(head.duration_bias.detach().numpy(), z["duration_bias"])
    np.testing.assert_array_equal(head.projection.weight.detach().numpy(), z["proj_weight"])
    assert "max_duration=12" in repr(head)


def test_score_gold_fails_loudly_off_gpu():
    cum = torch.zeros(2, 6, 3)
    with pytest.raises(RuntimeError, match="AMD GPU"):
        tsa.score_gold_vectorized(cum, torch.zeros(2, 5, dtype=torch.long), torch.tensor([5, 3]),
                                  torch.zeros(3, 3), torch.zeros(4, 3), 4)


def test_compute_edge_block_matches_oracle():
    g = torch.Generator().manual_seed(5)
    B, T, C, K = 2, 20, 3, 6
    cum = torch.randn(B, T + 1, C, generator=g).cumsum(1)
    tr = torch.randn(C, C, generator=g)
    db = torch.randn(K, C, generator=g)
    ps = torch.randn(B, T, C, generator=g)
    pe = torch.randn(B, T, C, generator=g)
    for t, k in [(3, 2), (10, 5), (0, 1)]:
        got = compute_edge_block_streaming(cum, tr, db, t, k, ps, pe)
        want = R.edge_blocks(cum, tr, db, torch.tensor([t]), torch.tensor([k]), ps, pe)[:, 0]
        assert torch.equal(got, want)


def test_segment_dataclass():
    s = tsa.Segment(start=3, end=7, label=2, score=1.5)
    assert s.duration == 5
    r = tsa.ViterbiResult(scores=torch.zeros(1), segments=[[s]])
    assert r.segments[0][0].label == 2


def test_kernel_timing_interface_without_gpu():
    lib = N.lib()
    n = lib.tsm_timing_kernel_count()
    names = [lib.tsm_timing_kernel_name(i).decode() for i in range(n)]
    assert "scan_fwd_kernel" in names and "marginal_kernel" in names and "viterbi_kernel" in names
    assert len(set(names)) == n
    assert lib.tsm_timing_kernel_name(n) is None and lib.tsm_timing_kernel_name(-1) is None
    # enabling and reading with nothing launched needs no device
    N.timing_enable(True)
    assert N.timing_read() == {}
    N.timing_enable(False)
    assert lib.tsm_timing_read(None, None, -1) == 1


def test_fast_path_is_planned_for_the_benchmark_shapes():
    """The log-semiring scans of the benchmark configurations run on the
    register-resident kernels (the generic kernels remain for the max
    semiring, very large label sets and tests)."""
    for B, T, C, K in ((1, 1_000_000, 24, 300), (4, 1000, 24, 100), (32, 10_000, 8, 1), (64, 8192, 32, 64)):
        assert N.plan_info(B, T, C, K)["fast"] == 1, (B, T, C, K)
