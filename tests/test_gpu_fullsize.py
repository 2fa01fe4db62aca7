"""The benchmark configurations at their full sizes (needs an MI355X; run with
``-m gpu``).

The full systems are too large for the CPU oracle to evaluate whole in a
test, so parity at full size is checked through what does not depend on size:

* C4 neighbour lists (7.1 M records) bit for bit against the oracle's builder;
* C4 per-atom energies against the oracle on clusters cut around chosen
  atoms: an EQ energy depends only on atoms within rc + 2 message cutoffs
  (6 + 6 + 6 Å) of its atom, so a non-periodic cluster of radius 18.5 Å gives
  that atom's exact periodic energy (likewise for MP, C3);
* C4 invariants: total force zero (Newton's third law over the records),
  symmetric virial (rotation invariance), structure energy equal to the sum
  of the per-atom energies, bitwise repeatability;
* C1 (512 atoms) and C2 (13,824 atoms) whole against the oracle;
* C5: cells of the 256-cell batch against the oracle cell by cell.
"""

import numpy as np
import pytest
import torch

from oracle import model as OM
from oracle import neighbors as ONB
from rune_amd import workloads as W
from tests.helpers import load_weights
from tests.test_gpu_parity import TOL, _nep_oracle, assert_within, check_against_oracle

pytestmark = pytest.mark.gpu

RECEPTIVE = 18.5   # Å: descriptor cutoff plus two message cutoffs, with margin


def _evaluator(kind):
    from rune_amd import _native as N
    from rune_amd.api import Evaluator
    p, w = load_weights(kind, torch.float32)
    return Evaluator(p, w, N.FAMILY_MOBIUS), p


@pytest.fixture(scope="module")
def c4():
    s = W.amorphous(seed=4)
    print("C4 generated:", len(s), "atoms", flush=True)
    return s


def test_c4_neighbor_list_bit_exact(c4):
    from rune_amd import _native as N
    ref = ONB.build(c4.positions, c4.cell, c4.pbc, 6.0, 5.0)
    nl = N.NeighborList().build(torch.as_tensor(c4.positions, device="cuda"), [0, len(c4)],
                                [c4.cell], [c4.pbc], 6.0, 5.0, 819, 819)
    out = {k: v.cpu().numpy() for k, v in nl.export().items()}
    print("C4 records:", nl.n_records, flush=True)
    assert nl.n_records == len(ref["neighbor"])
    np.testing.assert_array_equal(out["ptr"], ref["ptr"])
    np.testing.assert_array_equal(out["nbr"], ref["neighbor"])
    np.testing.assert_array_equal(out["shift"], ref["shift"])
    np.testing.assert_array_equal(out["vec"][:, :3], ref["vec32"])
    counts_a = np.bincount(ref["center"][ref["angular_mask"]], minlength=len(c4))
    np.testing.assert_array_equal(out["view"][:, 3] - out["view"][:, 2], counts_a)


@pytest.mark.parametrize("make", [lambda: W.fcc_alloy(seed=3),
                                  lambda: W.amorphous(seed=6, n_atoms=40_000)],
                         ids=["c3_19652", "amorphous_40000"])
def test_mid_size_neighbor_list_bit_exact(make):
    """Neighbour lists of the C3 cell (19,652 atoms) and a 40,000-atom
    amorphous cell bit for bit against the oracle's builder: atom counts
    above the single-workgroup scan (16,384), below C4's."""
    from rune_amd import _native as N
    s = make()
    print("mid-size cell:", len(s), "atoms", flush=True)
    ref = ONB.build(s.positions, s.cell, s.pbc, 6.0, 5.0)
    nl = N.NeighborList().build(torch.as_tensor(s.positions, device="cuda"), [0, len(s)],
                                [s.cell], [s.pbc], 6.0, 5.0, 819, 819)
    out = {k: v.cpu().numpy() for k, v in nl.export().items()}
    assert nl.n_records == len(ref["neighbor"])
    np.testing.assert_array_equal(out["ptr"], ref["ptr"])
    np.testing.assert_array_equal(out["nbr"], ref["neighbor"])
    np.testing.assert_array_equal(out["shift"], ref["shift"])
    np.testing.assert_array_equal(out["vec"][:, :3], ref["vec32"])
    counts_a = np.bincount(ref["center"][ref["angular_mask"]], minlength=len(s))
    np.testing.assert_array_equal(out["view"][:, 3] - out["view"][:, 2], counts_a)


def _cluster(s, i, radius):
    """Atoms within ``radius`` of atom i (minimum image of a cubic cell), atom i
    first, as a non-periodic structure."""
    L = np.diag(s.cell)
    d = s.positions - s.positions[i]
    d -= L * np.round(d / L)
    r = np.linalg.norm(d, axis=1)
    idx = np.argsort(r, kind="stable")
    idx = idx[r[idx] < radius]
    assert idx[0] == i
    box = 4.0 * radius
    return W.Structure(d[idx] + 0.5 * box, s.numbers[idx], np.eye(3) * box,
                       pbc=(False, False, False))


def _oracle_energy_of_first(kind, cl, types, dtype):
    p, w = load_weights(kind, dtype)
    nl = ONB.build(cl.positions, cl.cell, cl.pbc, p["rcut_radial"], p["rcut_angular"])
    sp = ONB.split(nl)
    mk = lambda k: OM.Edges(torch.as_tensor(sp[k][0]), torch.as_tensor(sp[k][1]),
                            torch.as_tensor(sp[k][2], dtype=dtype))
    r = OM.forward(w, p, torch.as_tensor(cl.positions, dtype=dtype),
                   torch.as_tensor(types, dtype=torch.long), [len(cl)], mk("radial"),
                   mk("angular"), compute_forces=False, compute_virial=False)
    return float(r["energies"][0])


def _check_cluster_energies(kind, ev, s, out, atoms):
    for i in atoms:
        cl = _cluster(s, i, RECEPTIVE)
        types = ev.types_of(cl.numbers)
        e64 = _oracle_energy_of_first(kind, cl, types, torch.float64)
        e32 = _oracle_energy_of_first(kind, cl, types, torch.float32)
        gpu = float(out["energies"][i])
        print(f"{kind} atom {i} ({len(cl)}-atom cluster): HIP - fp64 {gpu - e64:.2e}, "
              f"reference fp32 - fp64 {e32 - e64:.2e}, HIP - reference fp32 {gpu - e32:.2e}",
              flush=True)
        assert abs(gpu - e64) <= max(TOL[0], 2.0 * abs(e32 - e64))
        assert abs(gpu - e32) <= TOL[0] + abs(e32 - e64)


def test_c4_energies_and_invariants_at_full_size(c4):
    ev, _ = _evaluator("eq")
    out = ev.evaluate(c4)
    again = ev.evaluate(c4)
    for k in ("energies", "energy", "forces", "virial"):
        assert torch.equal(out[k], again[k]), k
    e = out["energies"].double().cpu().numpy()
    f = out["forces"].double().cpu().numpy()
    w = out["virial"].double().cpu().numpy()[0].reshape(3, 3)
    n = len(c4)
    assert abs(float(out["energy"][0]) - e.sum()) <= 1e-6 * np.abs(e).sum()
    net = np.abs(f.sum(axis=0)).max()
    print(f"C4: sum |F| {np.abs(f).sum():.3e}, |sum F| {net:.2e}, "
          f"|W - W^T| {np.abs(w - w.T).max():.2e}", flush=True)
    assert net <= 1e-6 * np.abs(f).sum()
    assert np.abs(w - w.T).max() <= TOL[2] * n
    _check_cluster_energies("eq", ev, c4, out, [0, 54321])


def test_c3_energies_at_full_size():
    ev, _ = _evaluator("mp")
    s = W.fcc_alloy()
    out = ev.evaluate(s)
    f = out["forces"].double().cpu().numpy()
    assert np.abs(f.sum(axis=0)).max() <= 1e-6 * np.abs(f).sum()
    _check_cluster_energies("mp", ev, s, out, [7, 12345])


def test_c1_whole_against_oracle():
    ev, _ = _evaluator("loc")
    s = W.si_diamond()
    out = ev.evaluate(s)
    check_against_oracle("loc", out, s, ev.types_of(s.numbers))


def test_c2_whole_against_oracle():
    from rune_amd import _native as N
    from rune_amd.api import Evaluator
    from rune_amd.nep.model import seeded_nep
    model = seeded_nep(seed=0)
    ev = Evaluator(model.params, model.state_dict(), N.FAMILY_NEP)
    s = W.rocksalt()
    out = ev.evaluate(s)
    r64 = _nep_oracle(model, s, torch.float64)
    assert_within(out, r64, _nep_oracle(model, s, torch.float32), len(s), f"C2 {len(s)}")


def test_c2_odd_atom_count_against_oracle():
    """The C2 cell without its last atom: 13,823 centres, so the last wave of
    the two-centres-per-wave descriptor kernels holds one centre."""
    from rune_amd import _native as N
    from rune_amd.api import Evaluator
    from rune_amd.nep.model import seeded_nep
    model = seeded_nep(seed=0)
    ev = Evaluator(model.params, model.state_dict(), N.FAMILY_NEP)
    c2 = W.rocksalt()
    s = W.Structure(c2.positions[:-1], c2.numbers[:-1], c2.cell)
    assert len(s) % 2 == 1
    out = ev.evaluate(s)
    r64 = _nep_oracle(model, s, torch.float64)
    assert_within(out, r64, _nep_oracle(model, s, torch.float32), len(s), f"C2-1 {len(s)}")


def test_sparse_local_cell_against_oracle():
    """A 8,193-atom amorphous cell at 0.025 atoms / A^3 (22 records per centre
    on average, 36 at most) with the Mobius-Local model: the
    two-centres-per-wave descriptor kernels with every invariant order
    (cubic ones included), and a last wave holding one centre."""
    ev, _ = _evaluator("loc")
    s = W.amorphous(seed=7, n_atoms=8193, density=0.025, dmin=1.8)
    out = ev.evaluate(s)
    check_against_oracle("loc", out, s, ev.types_of(s.numbers))


def test_c5_batch_cells_against_oracle():
    ev, _ = _evaluator("eq")
    cells = W.small_cells()
    out = ev.evaluate(cells)
    sp = np.concatenate([[0], np.cumsum([len(c) for c in cells])])
    for b in (0, 101, 255):
        c = cells[b]
        one = {"energies": out["energies"][sp[b]:sp[b + 1]],
               "forces": out["forces"][sp[b]:sp[b + 1]],
               "virial": out["virial"][b:b + 1], "energy": out["energy"][b:b + 1]}
        print(f"C5 cell {b}: {len(c)} atoms", flush=True)
        check_against_oracle("eq", one, c, ev.types_of(c.numbers))
