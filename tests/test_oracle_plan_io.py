"""Pins the plan-replay oracle (oracle/plan_io.py) and checks the trace-file layer (CPU only).

* A record written from the reference's own sparse-convex plan (the C1
  fixture) rebuilds that plan: keep, sources, parents and special ids
  exactly, the weights as their fp16 trace values, and the mass as one plus
  the per-parent sum of those weights (float64 brute force).
* Random records give plans whose keep and sources partition the tokens, whose
  parents point at the records' supports, and whose rejected rows stay kept.
* Trace files round-trip through the reference's {"layers": [...]} layout and
  malformed records are rejected before any GPU work.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import merging as om
from oracle import plan_io as opi
from tests.conftest import import_package

GOLDEN = Path(__file__).parent / "golden"
LAYOUT = dict(tokens_per_frame=261, patch_token_start=5)


@pytest.fixture(scope="module")
def fx():
    return np.load(GOLDEN / "fixtures_c1.npz")


def _reference_plan(fx):
    return (torch.from_numpy(fx["sc_keep"]), torch.from_numpy(fx["sc_source"]),
            torch.from_numpy(fx["sc_parent"]), torch.from_numpy(fx["sc_weight"]))


def test_record_of_the_reference_plan_rebuilds_it(fx):
    keep, source, parent, weight = _reference_plan(fx)
    record = opi.ttt_record_from_plan(keep, source, parent, weight, frames=4, **LAYOUT)
    assert record["source_ids"].dtype == torch.int32 and record["weights"].dtype == torch.float16
    out = opi.plan_from_ttt_record(record, **LAYOUT)
    assert torch.equal(out["keep"].reshape(-1), keep)
    assert torch.equal(out["source_original"].reshape(-1), source)
    assert torch.equal(out["parent_compact"].reshape(-1, 4), parent)
    assert torch.equal(out["special_compact"], torch.from_numpy(fx["sc_special_compact"]))
    w16 = weight.half().double()
    assert torch.equal(out["weights"].reshape(-1, 4).double(), w16)
    brute = torch.ones(keep.numel(), dtype=torch.float64).index_add_(0, parent.reshape(-1), w16.reshape(-1))
    mass = out["mass"].reshape(-1).double()
    assert (mass - brute).abs().max() <= 1e-6 * brute.max()
    # Against the reference's fp32-weight mass: each weight moved by at most 2^-11 of itself.
    ref = torch.from_numpy(fx["sc_mass"]).double()
    assert ((mass - ref).abs() <= 2.0 ** -11 * (ref - 1.0) + 1e-6).all()
    assert torch.allclose(out["log_mass"].reshape(-1).double(), mass.log(), rtol=1e-6, atol=0)


def _random_record(seed: int, frames: int, patches: int):
    g = torch.Generator().manual_seed(seed)
    n_patch = frames * patches
    perm = torch.randperm(n_patch, generator=g)
    n_src = n_patch // 3
    src, basis = perm[:n_src], perm[n_src:]
    support = basis[torch.randint(0, basis.numel(), (n_src, 4), generator=g)]
    accepted = torch.rand(n_src, generator=g) < 0.8
    e = -torch.rand(n_src, 4, generator=g).log()
    weights = (e / e.sum(-1, keepdim=True)).half()
    return dict(layer=seed, frames=frames, patches=patches, source_ids=src.int(),
                support_ids=support.int(), weights=weights, accepted=accepted)


@pytest.mark.parametrize("seed,frames", [(0, 2), (1, 3), (2, 5)])
def test_random_records_give_consistent_plans(seed, frames):
    pts, patches = 5, 64
    tpf = pts + patches
    record = _random_record(seed, frames, patches)
    out = opi.plan_from_ttt_record(record, tokens_per_frame=tpf, patch_token_start=pts)
    total = frames * tpf
    keep = out["keep"].reshape(-1)
    source = out["source_original"].reshape(-1)
    assert torch.equal(torch.cat([keep, source]).sort().values, torch.arange(total))
    assert (keep[1:] > keep[:-1]).all()
    ids = om.patch_ids(frames, tpf, pts).flatten()
    acc = record["accepted"]
    assert torch.equal(source, ids[record["source_ids"].long()[acc]])
    assert torch.equal(keep[out["parent_compact"].reshape(-1, 4)], ids[record["support_ids"].long()[acc]])
    assert torch.isin(ids[record["source_ids"].long()[~acc]], keep).all()
    assert torch.equal(keep[out["special_compact"]], out["special"])
    # A support that is itself an accepted source cannot stay physical.
    bad = dict(record)
    bad["support_ids"] = record["support_ids"].clone()
    first = int(acc.nonzero()[0])
    bad["support_ids"][first, 2] = record["source_ids"][first]
    with pytest.raises(RuntimeError, match="remain physical"):
        opi.plan_from_ttt_record(bad, tokens_per_frame=tpf, patch_token_start=pts)


def test_trace_file_round_trip_and_record_checks(tmp_path):
    pio = import_package("plan_io")
    records = [_random_record(s, 3, 64) for s in range(3)]
    path = tmp_path / "trace.pt"
    pio.save_ttt_trace(records, path)
    back = pio.read_ttt_trace(path)
    assert len(back) == 3
    for a, b in zip(records, back):
        assert a.keys() == b.keys()
        for key in a:
            assert torch.equal(a[key], b[key]) if isinstance(a[key], torch.Tensor) else a[key] == b[key]
    torch.save({"not_layers": 1}, tmp_path / "other.pt")
    with pytest.raises(ValueError, match="not a TTT trace"):
        pio.read_ttt_trace(tmp_path / "other.pt")
    kw = dict(tokens_per_frame=69, patch_token_start=5)
    with pytest.raises(ValueError, match="no 'accepted'"):
        pio.plan_from_ttt_record({k: v for k, v in records[0].items() if k != "accepted"}, **kw)
    with pytest.raises(ValueError, match="outside"):
        pio.plan_from_ttt_record(dict(records[0], source_ids=records[0]["source_ids"] + 1000), **kw)
    with pytest.raises(ValueError, match="support_ids \\[M,4\\]"):
        pio.plan_from_ttt_record(dict(records[0], support_ids=records[0]["support_ids"][:, :3]), **kw)
    with pytest.raises(ValueError, match="layout"):
        pio.plan_from_ttt_record(records[0], tokens_per_frame=70, patch_token_start=5)
