"""Seeded random shapes: HIP forward + backward against the fp64 oracle.

Each case draws B, T, C, K, ragged lengths, the semiring and optional boundary
projections, and compares log Z / the Viterbi score (1e-5 relative) and every
gradient (1e-5 relative + 1e-4 absolute) with `oracle.streaming_ref`'s fp64
restatement of the reference recursion (pytorch_reference.py:116-525).  The
plan variants run the same draws with more, shorter chunks (TSM_PLAN_P=8) and
with 8-lane label groups (TSM_FAST_J=8), so the chunk boundaries, the
speculation's verification and fix-up, and both lane layouts meet shapes that
the fixed-shape tests do not pick.
"""

import random

import pytest
import torch

from conftest import gpu_available
from oracle import streaming_ref as R

pytestmark = pytest.mark.gpu

if gpu_available():
    DEV = torch.device("cuda", 0)
else:  # collected on CPU, never run there
    DEV = None

import torch_semimarkov_amd as tsa  # noqa: E402

N_CASES = 16
VARIANTS = {
    "default": ({}, 64, 23),
    "p8": ({"TSM_PLAN_P": "8"}, 64, 29),
    "j8": ({"TSM_FAST_J": "8"}, 32, 31),
}


def draw(seed, case, cmax):
    rng = random.Random(seed * 1000 + case)
    C = rng.choice([c for c in (2, 3, 5, 8, 12, 16, 24, 33, 48, 64) if c <= cmax])
    K = rng.choice((1, 2, 3, 7, 16, 33, 60, 120, 200))
    T = rng.choice((5, 40, 150, 301, 520))
    B = rng.choice((1, 2, 3))
    sr = rng.choice(("log", "log", "max"))
    proj = rng.random() < 0.3
    L = [T] + [rng.randint(1, T) for _ in range(B - 1)]
    return B, T, C, K, sr, proj, L


@pytest.mark.parametrize("case", range(N_CASES))
@pytest.mark.parametrize("variant", list(VARIANTS))
def test_random_shapes_vs_fp64_oracle(variant, case, monkeypatch):
    env, cmax, seed = VARIANTS[variant]
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    B, T, C, K, sr, proj, L = draw(seed, case, cmax)
    print(f"{variant} case {case}: B={B} T={T} C={C} K={K} L={L} {sr} proj={proj}", flush=True)
    g = torch.Generator().manual_seed(seed * 1000 + case)
    cum = torch.zeros(B, T + 1, C)
    cum[:, 1:] = torch.randn(B, T, C, generator=g).cumsum(1)
    tr = 0.3 * torch.randn(C, C, generator=g)
    db = 0.3 * torch.randn(K, C, generator=g)
    ps = 0.1 * torch.randn(B, T, C, generator=g) if proj else None
    pe = 0.1 * torch.randn(B, T, C, generator=g) if proj else None
    lengths = torch.tensor(L)
    weights = torch.linspace(0.5, 2.0, B).double()

    def leaves(dev, dtype):
        return [None if x is None else x.to(dev, dtype).clone().requires_grad_(True) for x in (cum, tr, db, ps, pe)]

    c64, t64, b64, p64, e64 = leaves("cpu", torch.float64)
    want = R.streaming_oracle(c64, t64, b64, lengths, K, sr, p64, e64)
    ins64 = [x for x in (c64, t64, b64, p64, e64) if x is not None]
    gwant = torch.autograd.grad((want * weights).sum(), ins64)

    cd, td, bd, pd, ed = leaves(DEV, torch.float32)
    got = tsa.semi_crf_streaming_forward(cd, td, bd, lengths.to(DEV), K, semiring=sr, proj_start=pd, proj_end=ed)
    ins = [x for x in (cd, td, bd, pd, ed) if x is not None]
    ggot = torch.autograd.grad((got * weights.float().to(DEV)).sum(), ins)

    torch.testing.assert_close(got.double().cpu(), want.detach(), rtol=1e-5, atol=1e-5 * max(1.0, want.abs().max().item()))
    for name, a, b in zip(("cum_scores", "transition", "duration_bias", "proj_start", "proj_end"), ggot, gwant):
        torch.testing.assert_close(a.double().cpu(), b, rtol=1e-5, atol=1e-4, msg=lambda m, n=name: f"{n}: {m}")
