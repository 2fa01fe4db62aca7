"""Pin the neighbour-list oracle: literal reference cases, brute force, invariants."""

import numpy as np
import pytest

from oracle import neighbors as NB
from rune_amd import workloads as W


def _counts(nl, kind):
    return len(nl["center"][nl[f"{kind}_mask"]])


def test_reference_neighbor_frames_edge_counts():
    """rune tests/mobius_neighbor_check.py:24-83 with the counts asserted at :159-160."""
    cell = np.eye(3) * 30.0
    pos = np.array([[5., 5., 5.], [8.9, 5., 5.], [17., 17., 17.], [22., 17., 17.]])
    frames = []
    frames.append(pos.copy())
    pos[1, 0] = 8.7
    frames.append(pos.copy())
    pos[1, 0] = 8.45
    frames.append(pos.copy())
    pos[1, 0] = 8.95
    frames.append(pos.copy())
    pos[3, 0] = 20.7
    frames.append(pos.copy())
    radial, angular = [], []
    for f in frames:
        nl = NB.build(f, cell, (True,) * 3, 3.8, 3.5)
        radial.append(_counts(nl, "radial"))
        angular.append(_counts(nl, "angular"))
    assert radial == [0, 2, 2, 0, 2]
    assert angular == [0, 0, 2, 0, 0]


def test_one_atom_offsets_are_exact_fp64():
    """rune tests/test_calculators.py:57-69: offsets are exactly +-spacing."""
    spacing = 3.1234567890123
    nl = NB.build(np.array([[0.1, 0.2, 0.3]]), np.diag([spacing, 4.2, 5.3]), (True,) * 3,
                  3.5, 3.4)
    for kind in ("radial", "angular"):
        off = nl["offset"][nl[f"{kind}_mask"]]
        assert sorted(off[:, 0].tolist()) == [-spacing, spacing]


@pytest.mark.parametrize("seed", range(6))
def test_cell_list_equals_brute_force(seed):
    rng = np.random.default_rng(seed)
    a = rng.uniform(7.0, 13.0, 3)
    cell = np.diag(a) + rng.uniform(-1.5, 1.5, (3, 3)) * (1 - np.eye(3))
    n = int(rng.integers(20, 60))
    pos = rng.random((n, 3)) @ cell + rng.normal(0, 3.0, (n, 3))   # some outside the cell
    pbc = tuple(bool(x) for x in rng.integers(0, 2, 3)) if seed % 2 else (True,) * 3
    rc_r, rc_a = 4.0, 3.0
    b = NB.build(pos, cell, pbc, rc_r, rc_a, method="brute")
    c = NB.build(pos, cell, pbc, rc_r, rc_a, method="celllist")
    for k in ("ptr", "center", "neighbor", "shift", "n_short"):
        np.testing.assert_array_equal(b[k], c[k])
    np.testing.assert_array_equal(b["vec32"], c["vec32"])


def test_symmetry_and_distances():
    s = W.amorphous(seed=7, n_atoms=300)
    nl = NB.build(s.positions, s.cell, s.pbc, 6.0, 5.0)
    fwd = set(zip(nl["center"], nl["neighbor"], map(tuple, nl["shift"])))
    rev = set(zip(nl["neighbor"], nl["center"], map(tuple, -nl["shift"])))
    assert fwd == rev
    d = np.sqrt(nl["d2"])
    assert d.max() < 6.0 and d.min() >= 1.8 - 1e-9
    # angular list is a prefix of every centre's segment
    for i in range(len(s)):
        seg = nl["angular_mask"][nl["ptr"][i]:nl["ptr"][i + 1]]
        k = nl["n_short"][i]
        assert seg[:k].all() and not seg[k:].any()


def test_small_triclinic_cell_has_multiple_images():
    cell = np.array([[4.1, .1, .2], [.0, 4.3, .1], [.1, .0, 4.5]])
    frac = np.array([[.10, .13, .22], [.82, .21, .37], [.30, .75, .19], [.68, .63, .81]])
    nl = NB.build(frac @ cell, cell, (True,) * 3, 6.0, 5.0)
    pairs = list(zip(nl["center"], nl["neighbor"]))
    assert len(pairs) > len(set(pairs))      # same j through several images
    assert ((nl["center"] == nl["neighbor"]) & nl["shift"].any(1)).any()   # self images


def test_overflow_message():
    s = W.si_diamond(seed=1, reps=2)
    with pytest.raises(ValueError, match="exceeds max_neighbors=10"):
        NB.build(s.positions, s.cell, s.pbc, 6.0, 5.0, max_radial=10, max_angular=100)
