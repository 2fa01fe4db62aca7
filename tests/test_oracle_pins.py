"""Closed-form pins of the oracle's NEP network and flexible-ZBL pair rows (CPU).

* NEP per-element network (``rune/nep/model.py:157-170``): a literal nep.txt
  written out by hand here (not by any writer of this build), read by the
  drop-in reader (``rune/nep/model.py:284-489``; the file stores the hidden
  bias negated, ``:436-446``), then the oracle's ``nep_energies`` against
  ``E = sum_h w1[h] tanh(sum_k W0[h,k] q_k s_k - b_file[h]) - shared_bias``
  evaluated with ``math.tanh`` from the literal numbers.  An isolated atom has
  q = 0, so its energy is ``sum_h w1[h] tanh(-b_file[h]) - shared_bias`` and
  its force and virial vanish.
* Flexible ZBL (``rune/mobius/zbl.py:112-118``): the pair row of (t_i, t_j)
  is found by enumerating the upper triangle of the type pairs row-major
  (brute force, not the closed-form index), and the screened energy is
  evaluated with ``math.exp`` / ``math.cos``.
"""

import math

import numpy as np
import pytest
import torch

from oracle import model as OM
from oracle import neighbors as ONB
from oracle import tables as T
from rune_amd import workloads as W
from rune_amd.nep import plugin as NP

ELEMENTS = ["H", "O"]
HIDDEN = 2
Q = 6          # n_desc 2 + 2 * num_L (L = 1, 2)


def _literal_numbers():
    """Multiples of 1/8 (exact in float32), distinct per position."""
    w = {}
    k = 0

    def take(n):
        nonlocal k
        vals = [((k + i) * 5 % 17 - 8) * 0.125 for i in range(n)]
        k += n
        return vals

    for el in ELEMENTS:
        w[el] = {"w0": take(HIDDEN * Q), "b_file": take(HIDDEN), "w1": take(HIDDEN)}
    w["shared"] = 0.375
    w["c_radial"] = take(16)
    w["c_angular"] = take(16)
    w["scaler"] = [0.5 + 0.125 * i for i in range(Q)]
    return w


def _literal_text(w, zbl=None):
    lines = [("nep4_zbl" if zbl else "nep4") + " 2 H O"]
    if zbl:
        lines.append(f"zbl {zbl[0]} {zbl[1]}")
    lines += ["cutoff 5.0 4.0 20 20", "n_max 1 1", "basis_size 1 1", "l_max 2 0 0", "ANN 2 0"]
    vals = []
    for el in ELEMENTS:
        vals += w[el]["w0"] + w[el]["b_file"] + w[el]["w1"]
    vals.append(w["shared"])
    vals += w["c_radial"] + w["c_angular"] + w["scaler"]
    lines += [f"{v:18.10e}" for v in vals]
    return "\n".join(lines) + "\n"


def _closed_form(w, el, q):
    e = -w["shared"]
    for h in range(HIDDEN):
        z = sum(w[el]["w0"][h * Q + k] * q[k] * w["scaler"][k] for k in range(Q))
        e += w[el]["w1"][h] * math.tanh(z - w[el]["b_file"][h])
    return e


@pytest.fixture()
def literal_model(tmp_path):
    w = _literal_numbers()
    path = tmp_path / "nep.txt"
    path.write_text(_literal_text(w))
    return w, NP.load_model(path)


def test_nep_network_matches_closed_form(literal_model):
    w, model = literal_model
    assert model.params["n_desc_radial"] + model.params["n_desc_angular"] * model.num_L == Q
    sd = {k: v.double() if v.is_floating_point() else v for k, v in model.state_dict().items()}
    rng = np.random.default_rng(5)
    q = rng.normal(size=(6, Q))
    types = torch.tensor([0, 1, 1, 0, 1, 0])
    empty = torch.zeros(0, dtype=torch.long)
    e = OM.nep_energies(sd, model.params, torch.as_tensor(q), types, empty, empty,
                        torch.zeros((0, 3), dtype=torch.float64))
    for a in range(6):
        expect = _closed_form(w, ELEMENTS[int(types[a])], q[a])
        assert abs(e[a].item() - expect) < 1e-12, (a, e[a].item(), expect)


def test_nep_isolated_atoms_closed_form(literal_model):
    """q = 0 without neighbours: E = sum_h w1 tanh(-b_file) - shared_bias, F = W = 0."""
    w, model = literal_model
    p = model.params
    sd = {k: v.double() if v.is_floating_point() else v for k, v in model.state_dict().items()}
    s = W.Structure(np.array([[1.0, 1.0, 1.0], [40.0, 1.0, 1.0], [1.0, 40.0, 1.0]]),
                    np.array([1, 8, 1]), np.zeros((3, 3)), pbc=(False, False, False))
    nl = ONB.build(s.positions, s.cell, s.pbc, p["rcut_radial"], p["rcut_angular"])
    assert len(nl["center"]) == 0
    sp = ONB.split(nl)
    mk = lambda k: OM.Edges(torch.as_tensor(sp[k][0]), torch.as_tensor(sp[k][1]),
                            torch.as_tensor(sp[k][2]))
    out = OM.nep_forward(sd, p, torch.as_tensor(s.positions), torch.tensor([0, 1, 0]), [3],
                         mk("radial"), mk("angular"))
    for a, el in enumerate(["H", "O", "H"]):
        expect = _closed_form(w, el, [0.0] * Q)
        assert abs(out["energies"][a].item() - expect) < 1e-12
    assert torch.count_nonzero(out["forces"]) == 0
    assert torch.count_nonzero(out["virial"]) == 0


def test_nep_writer_stores_bias_negated(literal_model, tmp_path):
    """Writing the read model back gives the literal file's numbers (``:535-540``)."""
    w, model = literal_model
    path = NP.export_model(model, tmp_path / "back")
    numbers = [float(x) for line in path.read_text().splitlines()[6:] for x in line.split()]
    expect = [float(x) for line in _literal_text(w).splitlines()[6:] for x in line.split()]
    assert numbers == expect


def _pair_rows(n):
    return [(lo, hi) for lo in range(n) for hi in range(lo, n)]


def _flexible_table(n):
    rows = []
    for r in range(n * (n + 1) // 2):
        coeff = []
        for k in range(4):
            coeff += [0.1 * (k + 1) + 0.01 * r, 0.5 * (k + 1) + 0.02 * r]
        rows.append([0.5 + 0.1 * r, 2.0 + 0.1 * r] + coeff)
    return np.array(rows, dtype=np.float32).astype(np.float64)


@pytest.mark.parametrize("ti,tj", [(a, b) for a in range(3) for b in range(3)])
def test_flexible_zbl_pair_row(ti, tj):
    numbers = [26.0, 6.0, 8.0]
    table = _flexible_table(3)
    row = table[_pair_rows(3).index((min(ti, tj), max(ti, tj)))]
    d = 1.2
    zi, zj = numbers[ti], numbers[tj]
    a_inv = (zi ** 0.23 + zj ** 0.23) * T.ZBL_A_INV_FACTOR
    phi = sum(row[2 + 2 * k] * math.exp(-row[3 + 2 * k] * d * a_inv) for k in range(4))
    cut = 0.5 * math.cos(math.pi * (d - row[0]) / (row[1] - row[0])) + 0.5
    expect = 0.5 * T.K_C_SP * zi * zj * phi / d * cut
    types = torch.tensor([ti, tj])
    vec = torch.tensor([[0.0, d, 0.0]], dtype=torch.float64)
    e = OM.zbl_energy(vec, torch.tensor([0]), torch.tensor([1]), types, 2,
                      torch.tensor(numbers), {"rc_inner": 0.0, "rc_outer": 0.0, "flexible": True},
                      3, torch.as_tensor(table))
    assert abs(e[0].item() - expect) <= 1e-12 * abs(expect)
    assert e[1].item() == 0.0
