"""Verlet-skin reuse of the neighbour lists (``rune_nlist_update``) against a
fresh ``rune_nlist_build`` at every step of a random walk of the atoms (needs
an MI355X; run with ``-m gpu``).

The reference's GPUMD evaluator keeps a candidate list at rc + 1 A and reuses
it while every atom moved less than skin / 2 (rune/mobius/src/mobius.cu:241-271,
:334-402).  Here reuse must be invisible: the records of every call are
compared bit for bit with a fresh build on the same positions and with the
oracle's canonical lists (``oracle/neighbors.py``), and the model outputs
through both lists must be identical.
"""

import numpy as np
import pytest
import torch

from oracle import neighbors as ONB
from rune_amd import workloads as W
from tests.helpers import load_weights

pytestmark = pytest.mark.gpu

RC_R, RC_A, SKIN, LIMIT = 6.0, 5.0, 1.0, 4000


def _system(case):
    if case == "amorphous":
        structs = [W.amorphous(seed=31, n_atoms=1500)]
        pbc = [np.ones(3, np.int32)]
    elif case == "small_cells":
        structs = W.small_cells(seed=32, n_cells=6)
        pbc = [np.ones(3, np.int32)] * len(structs)
    else:   # a cluster: no periodic direction, the cell only bounds the binning
        structs = [W.amorphous(seed=33, n_atoms=400)]
        pbc = [np.zeros(3, np.int32)]
    pos = np.concatenate([s.positions for s in structs])
    sp = np.concatenate([[0], np.cumsum([len(s) for s in structs])]).astype(np.int64)
    cells = np.stack([np.asarray(s.cell, np.float64) for s in structs])
    return structs, pos, sp, cells, np.stack(pbc)


def _assert_same_records(upd, ref):
    assert upd.n_records == ref.n_records
    a, b = upd.export(), ref.export()
    for k in ("ptr", "view", "nbr", "shift"):
        assert torch.equal(a[k], b[k]), k
    assert torch.equal(a["vec"].view(torch.int32), b["vec"].view(torch.int32))


def _assert_matches_oracle(upd, pos, sp, cells, pbc):
    """Records of every structure against the oracle's list, bit for bit."""
    out = {k: v.cpu().numpy() for k, v in upd.export().items()}
    for k in range(len(sp) - 1):
        a, b = int(sp[k]), int(sp[k + 1])
        ref = ONB.build(pos[a:b], cells[k], tuple(bool(x) for x in pbc[k]), RC_R, RC_A)
        lo, hi = out["ptr"][a], out["ptr"][b]
        np.testing.assert_array_equal(out["ptr"][a:b + 1] - lo, ref["ptr"])
        np.testing.assert_array_equal(out["nbr"][lo:hi] - a, ref["neighbor"])
        np.testing.assert_array_equal(out["shift"][lo:hi], ref["shift"])
        np.testing.assert_array_equal(out["vec"][lo:hi, :3], ref["vec32"])


@pytest.mark.parametrize("case", ["amorphous", "small_cells", "cluster"])
def test_skin_reuse_matches_fresh_build(case):
    from rune_amd import _native as N
    _, pos, sp, cells, pbc = _system(case)
    rng = np.random.default_rng(34)
    upd, ref = N.NeighborList(), N.NeighborList()
    searched = []
    for step in range(14):
        if step:
            pos = pos + rng.normal(0.0, 0.05, pos.shape)
        t = torch.as_tensor(pos, device="cuda")
        searched.append(upd.update(t, sp, cells, pbc, RC_R, RC_A, LIMIT, LIMIT, SKIN))
        ref.build(t, sp, cells, pbc, RC_R, RC_A, LIMIT, LIMIT)
        _assert_same_records(upd, ref)
        _assert_matches_oracle(upd, pos, sp, cells, pbc)
    print(case, "searched at steps", [k for k, s in enumerate(searched) if s], flush=True)
    # the first call searches; small moves reuse; the walk outgrows skin / 2
    assert searched[0] and not searched[1] and any(searched[2:])
    # a changed cell (positions scaled with it) forces a search
    t = torch.as_tensor(pos * 1.01, device="cuda")
    assert upd.update(t, sp, cells * 1.01, pbc, RC_R, RC_A, LIMIT, LIMIT, SKIN)
    ref.build(t, sp, cells * 1.01, pbc, RC_R, RC_A, LIMIT, LIMIT)
    _assert_same_records(upd, ref)
    _assert_matches_oracle(upd, pos * 1.01, sp, cells * 1.01, pbc)


def test_skin_reuse_reports_overflow_like_build():
    from rune_amd import _native as N
    _, pos, sp, cells, pbc = _system("amorphous")
    t = torch.as_tensor(pos, device="cuda")
    upd = N.NeighborList()
    assert upd.update(t, sp, cells, pbc, RC_R, RC_A, LIMIT, LIMIT, SKIN)
    with pytest.raises(ValueError, match="exceeds max_neighbors=20"):
        upd.update(t, sp, cells, pbc, RC_R, RC_A, 20, LIMIT, SKIN)
    # the handle recovers on the next valid call
    assert upd.update(t, sp, cells, pbc, RC_R, RC_A, LIMIT, LIMIT, SKIN)


def test_model_through_reused_lists_is_bitwise_equal():
    from rune_amd import _native as N
    from rune_amd.api import Evaluator
    p, w = load_weights("eq", torch.float32)
    ev = Evaluator(p, w, N.FAMILY_MOBIUS)
    s = W.amorphous(seed=35, n_atoms=300)
    types = torch.as_tensor(ev.types_of(s.numbers), device="cuda")
    sp, cells, pbc = [0, len(s)], [s.cell], [np.ones(3, np.int32)]
    rc = (p["rcut_radial"], p["rcut_angular"], p["max_neighbors_radial"],
          p["max_neighbors_angular"])
    rng = np.random.default_rng(36)
    upd, ref = N.NeighborList(), N.NeighborList()
    pos = s.positions
    reused = 0
    for step in range(4):
        if step:
            pos = pos + rng.normal(0.0, 0.03, pos.shape)
        t = torch.as_tensor(pos, device="cuda")
        reused += not upd.update(t, sp, cells, pbc, *rc, SKIN)
        ref.build(t, sp, cells, pbc, *rc)
        a = ev.native.compute(upd, types, 1)
        b = ev.native.compute(ref, types, 1)
        for k in ("energies", "energy", "forces", "virial"):
            assert torch.equal(a[k], b[k]), (step, k)
    assert reused >= 1
