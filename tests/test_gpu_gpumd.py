"""GPUMD-style per-atom outputs (``rune_model_compute_gpumd``): fp64 arrays in
GPUMD's layout, accumulated like GPUMD's potentials
(rune/mobius/src/force.cu:47-84), and the heat-current support flag
(rune/mobius/src/mobius.cuh:18).  Needs an MI355X; run with ``-m gpu``."""

import numpy as np
import pytest
import torch

from rune_amd import workloads as W
from tests.helpers import load_weights

pytestmark = pytest.mark.gpu

A = [0, 1, 2, 0, 0, 1, 1, 2, 2]
B = [0, 1, 2, 1, 2, 2, 0, 0, 1]


@pytest.mark.parametrize("name, heat", [("loc", True), ("mp", False), ("eq", False)])
def test_gpumd_outputs_follow_gpumd_layout(name, heat):
    from rune_amd import _native as N
    from rune_amd.api import Evaluator
    p, w = load_weights(name, torch.float32)
    ev = Evaluator(p, w, N.FAMILY_MOBIUS)
    assert ev.native.supports_heat_current() == heat
    s = W.amorphous(seed=51, n_atoms=200)
    types = torch.as_tensor(ev.types_of(s.numbers), device="cuda")
    nl = N.NeighborList().build(torch.as_tensor(s.positions, device="cuda"), [0, len(s)],
                                [s.cell], [np.ones(3, np.int32)], p["rcut_radial"],
                                p["rcut_angular"], p["max_neighbors_radial"],
                                p["max_neighbors_angular"])
    ref = ev.native.compute(nl, types, 1, True, True, atom_virial=True)
    n = len(s)
    dev = "cuda"
    pot = torch.ones(n, dtype=torch.float64, device=dev)
    force = torch.full((3 * n,), 2.0, dtype=torch.float64, device=dev)
    vir = torch.full((9 * n,), 3.0, dtype=torch.float64, device=dev)
    ev.native.compute_gpumd(nl, types, pot, force, vir)
    assert torch.equal(pot, 1.0 + ref["energies"].double())
    assert torch.equal(force.view(3, n), 2.0 + ref["forces"].double().T)
    wat = ref["atom_virial"].double().view(n, 3, 3)
    expect = torch.stack([wat[:, B[k], A[k]] for k in range(9)])
    assert torch.equal(vir.view(9, n), 3.0 + expect)
    # the nine arrays sum to the transposed structure virial (W_ab = -sum g_a r_b)
    total = (vir.view(9, n) - 3.0).sum(1)
    wsum = ref["virial"][0].double().view(3, 3)
    got = torch.zeros(3, 3, dtype=torch.float64, device=dev)
    for k in range(9):
        got[A[k], B[k]] = total[k]
    torch.testing.assert_close(got, wsum.T, rtol=1e-5, atol=1e-4)


def test_nep_supports_heat_current():
    from rune_amd import _native as N
    from rune_amd.nep.model import seeded_nep
    model = seeded_nep(seed=9)
    native = N.NativeModel(model.params, model.state_dict(), N.FAMILY_NEP)
    assert native.supports_heat_current()
