"""Writes the benchmark-configuration fixtures ``tests/golden/config_cfg{1,3,4,5}.npz``.

    python tests/golden/make_config_fixtures.py [cfg1 cfg3 cfg4 cfg5]

Each file holds OUTPUTS of the fp64 oracle (and, for the Viterbi
configurations, of the fp32 restatement of the reference's Viterbi) on the
exact synthetic inputs that ``bench.py`` draws for that configuration
(``bench.make_inputs`` / ``bench.make_head_inputs``: seeded
``torch.Generator`` draws in a fixed order), plus an input checksum.  The
inputs themselves are not stored: the GPU tests draw them again from the seed
and assert the checksum first, so a changed draw fails loudly instead of
comparing different problems.

The oracle is ``oracle/cref.py`` (the C restatement ``oracle/semimarkov_ref.c``,
pinned against ``oracle/streaming_ref.py`` in ``tests/test_oracle.py``) and, for
the head's gold-path score, ``oracle/streaming_ref.score_gold``.  Run time in
the build container (8 cores): cfg1 seconds, cfg3 about 3 minutes, cfg4 about
20 s, cfg5 about 10 minutes.

What each file holds (all fp64 unless stated):

* ``config_cfg1``: the head ``SemiMarkovCRFHead(24, 100, 512)`` loss
  ``mean_b(log Z_b - gold_b)`` and its gradients w.r.t. ``transition``,
  ``duration_bias``, ``projection.weight`` / ``.bias``, and the expected label
  occupancy that the bias gradient is a difference of; ``log Z``; the Viterbi
  score (``decode``) and its segments, with the smallest nonzero runner-up gap
  and the number of exact ties along each backtrace.
* ``config_cfg3`` (B=1, T=10^6, C=24, K=300): log Z, the max-semiring score,
  ``grad_transition``, ``grad_duration_bias`` and ``grad_cum`` at 4102 sampled
  rows (fp32), for ``grad_output = 1``.
* ``config_cfg4`` (64 ragged sequences, C=32, K=64): Viterbi scores and a
  SHA-256 of each sequence's segments, (a) from the fp32 restatement of the
  reference's recursion (bit-identical to the reference) and (b) from the fp64
  recursion, whose segments are hashed in canonical form (runs of one label
  with their durations sorted: reordering the segment durations of a run
  leaves the score unchanged exactly), with each path's smallest nonzero
  runner-up gap and exact-tie count.
* ``config_cfg5`` (B=8, T=5*10^4, C=128, K=500): log Z, ``grad_transition``,
  ``grad_duration_bias`` and ``grad_cum`` at 68 sampled rows per sequence
  (fp32), for ``grad_output = 1``.
"""

from __future__ import annotations

import hashlib
import os
import sys
import time

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for _p in (ROOT, os.path.join(ROOT, "torch-semimarkov_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)


# --------------------------------------------------------------------------- shared helpers (tests import these)
def input_checksum(*arrays) -> np.ndarray:
    """Per array: fp64 sum, sum of squares and an index-weighted sum."""
    out = []
    for a in arrays:
        x = a.detach().cpu().numpy() if hasattr(a, "detach") else np.asarray(a)
        x = x.astype(np.float64).ravel()
        w = (np.arange(x.size) % 997 + 1) / 997.0
        out += [x.sum(), (x * x).sum(), (x * w).sum()]
    return np.array(out)


def canonical_runs(segs):
    """Segments (start, end, label, prev) -> runs of one label, each as
    (start, end, label, sorted durations).  Two segmentations with the same
    canonical form have exactly the same score."""
    out = []
    i = 0
    while i < len(segs):
        j = i
        while j + 1 < len(segs) and segs[j + 1][2] == segs[i][2]:
            j += 1
        durs = tuple(sorted(int(s[1]) - int(s[0]) + 1 for s in segs[i : j + 1]))
        out.append((int(segs[i][0]), int(segs[j][1]), int(segs[i][2]), durs))
        i = j + 1
    return out


def seg_hash(segs) -> bytes:
    """SHA-256 of a segment list (start, end, label, prev), first segment first."""
    a = np.asarray([tuple(int(v) for v in s) for s in segs], dtype=np.int32).reshape(-1, 4)
    return hashlib.sha256(a.tobytes()).digest()


def canonical_hash(segs) -> bytes:
    flat = []
    for s, e, c, durs in canonical_runs(segs):
        flat += [s, e, c, len(durs)] + list(durs)
    return hashlib.sha256(np.asarray(flat, dtype=np.int32).tobytes()).digest()


def sample_rows(T: int, n: int, seed: int) -> np.ndarray:
    """Sorted sample of n positions in [0, T] plus both ends and their neighbours."""
    rng = np.random.default_rng(seed)
    idx = rng.choice(T + 1, size=min(n, T + 1), replace=False)
    idx = np.concatenate([idx, [0, 1, 2, T - 2, T - 1, T]])
    return np.unique(np.clip(idx, 0, T)).astype(np.int64)


def fixture_path(name: str) -> str:
    return os.path.join(HERE, f"config_{name}.npz")


# --------------------------------------------------------------------------- generators
def make_cfg1():
    import bench
    from oracle import cref
    from oracle import streaming_ref as R

    cfg, head, h, L, labels = bench.make_head_inputs()
    B, T, C, K = cfg["B"], cfg["T"], cfg["C"], cfg["K"]
    W = head.projection.weight.detach().double()
    bl = head.projection.bias.detach().double()
    tr = head.transition.detach().double()
    db = head.duration_bias.detach().double()
    h64 = h.double()
    scores = h64 @ W.T + bl
    cum = torch.zeros(B, T + 1, C, dtype=torch.float64)
    cum[:, 1:] = torch.cumsum(scores, dim=1)
    res = cref.backward(cum, tr, db, L, K)
    logZ = res["logZ"]
    # gold-path score and its gradients (fp64 autograd through the restatement)
    cum_g = cum.clone().requires_grad_(True)
    tr_g = tr.clone().requires_grad_(True)
    db_g = db.clone().requires_grad_(True)
    gold = R.score_gold(cum_g, labels, L, tr_g, db_g, K)
    gcum_gold, gtr_gold, gdb_gold = torch.autograd.grad(gold.sum(), [cum_g, tr_g, db_g])
    # loss = mean_b(logZ_b - gold_b)
    d_cum = (torch.from_numpy(res["grad_cum"]) - gcum_gold) / B
    d_tr = (torch.from_numpy(res["grad_transition"]).sum(0) - gtr_gold) / B
    d_db = (torch.from_numpy(res["grad_duration_bias"]).sum(0) - gdb_gold) / B
    # cum[u] = sum_{t < u} scores[t]  =>  d scores[t] = sum_{u > t} d cum[u]
    d_scores = torch.flip(torch.cumsum(torch.flip(d_cum[:, 1:], [1]), 1), [1])
    d_W = torch.einsum("btc,bth->ch", d_scores, h64)
    d_b = d_scores.sum((0, 1))
    # the scale of the projection-bias gradient: the expected occupancy of each label,
    # sum_b sum_t d log Z_b / d scores[b, t, c] / B = sum_b sum_u u * d log Z_b / d cum[b, u, c] / B
    occ = (np.arange(T + 1)[None, :, None] * res["grad_cum"]).sum((0, 1)) / B
    vit = cref.viterbi(cum, tr, db, L, K, dtype=np.float64)
    segs = vit["segments"]
    np.savez_compressed(
        fixture_path("cfg1"),
        checksum=input_checksum(h, labels, head.transition, head.duration_bias, head.projection.weight,
                                head.projection.bias),
        logZ=logZ, gold=gold.detach().numpy(), loss=np.float64((logZ - gold.detach().numpy()).mean()),
        grad_transition=d_tr.numpy(), grad_duration_bias=d_db.numpy(), grad_proj_weight=d_W.numpy(),
        grad_proj_bias=d_b.numpy(), proj_bias_scale=occ,
        viterbi_score=vit["score"], viterbi_nseg=np.array([len(s) for s in segs], dtype=np.int32),
        viterbi_segments=np.concatenate([np.asarray(s, dtype=np.int32).reshape(-1, 4) for s in segs]),
        viterbi_min_gap=vit["min_gap"], viterbi_n_ties=vit["n_ties"],
    )


def make_scan_fixture(name: str, rows_per_seq: int):
    import bench
    from oracle import cref

    cfg, cum, tr, db, L = bench.make_inputs(name)
    B, T, C, K = cfg["B"], cfg["T"], cfg["C"], cfg["K"]
    t0 = time.time()
    res = cref.backward(cum, tr, db, L, K)
    print(f"{name}: backward {time.time() - t0:.1f} s", flush=True)
    idx = np.stack([sample_rows(T, rows_per_seq, cfg["seed"] + b) for b in range(B)]) if B > 1 else \
        sample_rows(T, rows_per_seq, cfg["seed"])[None]
    n = min(len(i) for i in idx)
    idx = np.stack([i[np.linspace(0, len(i) - 1, n).round().astype(int)] for i in idx])
    rows = np.stack([res["grad_cum"][b, idx[b]] for b in range(B)]).astype(np.float32)
    out = dict(
        checksum=input_checksum(cum, tr, db, L), logZ=res["logZ"],
        grad_transition=res["grad_transition"].sum(0), grad_duration_bias=res["grad_duration_bias"].sum(0),
        grad_cum_rows_idx=idx, grad_cum_rows=rows,
    )
    if name == "cfg3":
        t0 = time.time()
        out["max_score"] = cref.forward(cum, tr, db, L, K, "max")
        print(f"{name}: max forward {time.time() - t0:.1f} s", flush=True)
    np.savez_compressed(fixture_path(name), **out)


def make_cfg4():
    import bench
    from oracle import cref

    cfg, cum, tr, db, L = bench.make_inputs("cfg4")
    K = cfg["K"]
    v32 = cref.viterbi(cum, tr, db, L, K, dtype=np.float32)
    v64 = cref.viterbi(cum, tr, db, L, K, dtype=np.float64)
    np.savez_compressed(
        fixture_path("cfg4"),
        checksum=input_checksum(cum, tr, db, L),
        f32_score=v32["score"], f32_nseg=np.array([len(s) for s in v32["segments"]], dtype=np.int32),
        f32_hash=np.stack([np.frombuffer(seg_hash(s), dtype=np.uint8) for s in v32["segments"]]),
        f64_score=v64["score"],
        f64_canonical_hash=np.stack([np.frombuffer(canonical_hash(s), dtype=np.uint8) for s in v64["segments"]]),
        f64_min_gap=v64["min_gap"], f64_n_ties=v64["n_ties"],
    )


def main(names):
    torch.set_num_threads(max(1, min(os.cpu_count() or 1, 16)))
    for name in names:
        t0 = time.time()
        if name == "cfg1":
            make_cfg1()
        elif name == "cfg3":
            make_scan_fixture("cfg3", 4096)
        elif name == "cfg4":
            make_cfg4()
        elif name == "cfg5":
            make_scan_fixture("cfg5", 64)
        else:
            raise SystemExit(f"unknown configuration {name!r}")
        print(f"{name}: wrote {fixture_path(name)} in {time.time() - t0:.1f} s", flush=True)


if __name__ == "__main__":
    main(sys.argv[1:] or ["cfg1", "cfg4", "cfg3", "cfg5"])
