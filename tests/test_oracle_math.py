"""Closed-form and invariance pins of the CPU oracle (independent of the golden files)."""

import math

import numpy as np
import pytest
import torch

from oracle import model as OM
from oracle import neighbors as ONB
from oracle import tables as T
from rune_amd import workloads as W


def test_chebyshev_closed_form_and_derivative():
    r = torch.linspace(0.3, 5.9, 41, dtype=torch.float64)
    rc = 6.0
    f, fp = OM.chebyshev_with_derivative(r, rc, 9)
    fc = 0.5 * torch.cos(math.pi * r / rc) + 0.5
    x = 2 * (r / rc - 1) ** 2 - 1
    for k in range(9):
        expect = fc if k == 0 else 0.5 * (torch.cos(k * torch.arccos(x)) + 1) * fc
        torch.testing.assert_close(f[:, k], expect, rtol=1e-12, atol=1e-12)
    h = 1e-6
    fph, _ = OM.chebyshev_with_derivative(r + h, rc, 9)
    fmh, _ = OM.chebyshev_with_derivative(r - h, rc, 9)
    torch.testing.assert_close(fp, (fph - fmh) / (2 * h), rtol=1e-6, atol=1e-8)
    masked = OM.chebyshev_masked(torch.tensor([7.0], dtype=torch.float64), rc, 4)
    assert torch.count_nonzero(masked) == 0


def _legendre(L, x):
    p0, p1 = np.ones_like(x), x
    if L == 0:
        return p0
    for n in range(1, L):
        p0, p1 = p1, ((2 * n + 1) * x * p1 - n * p0) / (n + 1)
    return p1


@pytest.mark.parametrize("L", range(1, 9))
def test_angular_basis_addition_theorem(L):
    """sum_m w_m b_m(u) b_m(v) = (2L+1)/(4 pi) P_L(u.v), w_0 = C3B_0, w_m = 2 C3B_m."""
    rng = np.random.default_rng(L)
    u = rng.normal(size=(20, 3))
    v = rng.normal(size=(20, 3))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    v /= np.linalg.norm(v, axis=1, keepdims=True)
    Z = OM.z_tables(None, torch.float64)
    bu = OM.angular_basis(torch.as_tensor(u), L, Z).numpy()
    bv = OM.angular_basis(torch.as_tensor(v), L, Z).numpy()
    a, b = L * L - 1, (L + 1) ** 2 - 1
    w = np.array(T.C3B[a:b]) * 2.0
    w[0] *= 0.5
    lhs = (bu[:, a:b] * bv[:, a:b] * w).sum(1)
    rhs = (2 * L + 1) / (4 * math.pi) * _legendre(L, (u * v).sum(1))
    np.testing.assert_allclose(lhs, rhs, rtol=1e-11, atol=1e-12)


def test_zbl_closed_form():
    """One Si-Si pair at 1.5 Å inside the taper of [1, 2] (rune/mobius/zbl.py:92-141)."""
    d = 1.5
    z = 14.0
    a_inv = (2 * z ** 0.23) * T.ZBL_A_INV_FACTOR
    # the reference stores the universal coefficients as a float32 buffer (zbl.py:41-44)
    coeffs = [(float(np.float32(a)), float(np.float32(b))) for a, b in T.UNIVERSAL_ZBL]
    phi = sum(a * math.exp(-b * d * a_inv) for a, b in coeffs)
    cut = 0.5 * math.cos(math.pi * (d - 1.0) / 1.0) + 0.5
    expect = 0.5 * T.K_C_SP * z * z * phi / d * cut
    vec = torch.tensor([[d, 0.0, 0.0]], dtype=torch.float64)
    e = OM.zbl_energy(vec, torch.tensor([0]), torch.tensor([1]), torch.tensor([0, 0]), 2,
                      torch.tensor([14.0]), {"rc_inner": 1.0, "rc_outer": 2.0, "flexible": False},
                      1)
    assert abs(e[0].item() - expect) < 1e-12 * expect
    assert e[1].item() == 0.0


def _small(kind, seed=11):
    from rune_amd.mobius.model import Mobius
    from rune_amd.mobius.plugin import resolve_params
    values = {"elements": ["Fe", "C"], "hidden_dim": 8, "blocks": 1, "ffn_dim": 12,
              "message_layers": 2, "message_dim": 8, "message_groups": 2, "pair_dim": 3,
              "vector_channels": 2, "message_basis_size": 3, "rcut_radial": 4.8,
              "rcut_angular": 4.4, "n_max_radial": 1, "n_max_angular": 1,
              "basis_size_radial": 2, "basis_size_angular": 2, "l_max": 4, "l_max_4body": 2,
              "l_max_5body": 1, "has_q_112": 1, "has_q_123": 1, "has_q_233": 1, "has_q_134": 1,
              "zbl": [0.8, 1.6]}
    if kind == "local":
        values["message_layers"] = 0
    if kind == "eq":
        values.update(message_mode="equivariant", equivariant_channels=3)
    torch.manual_seed(seed)
    model = Mobius(resolve_params(values))
    return model.params, {k: v.double() for k, v in model.state_dict().items()}


def _cell():
    cell = np.array([[3.9, 0.1, 0.2], [0.0, 4.1, 0.1], [0.1, 0.0, 4.3]])
    frac = np.array([[.10, .13, .22], [.82, .21, .37], [.30, .75, .19], [.68, .63, .81]])
    return W.Structure(frac @ cell, np.array([26, 6, 26, 6]), cell)


def _edges(s, p, rot=None):
    pos = s.positions if rot is None else s.positions @ rot.T
    cell = s.cell if rot is None else s.cell @ rot.T
    nl = ONB.build(pos, cell, s.pbc, p["rcut_radial"], p["rcut_angular"])
    sp = ONB.split(nl)
    mk = lambda k: OM.Edges(torch.as_tensor(sp[k][0]), torch.as_tensor(sp[k][1]),
                            torch.as_tensor(sp[k][2]))
    return torch.as_tensor(pos), mk("radial"), mk("angular")


@pytest.mark.parametrize("kind", ["local", "mp", "eq"])
def test_contraction_equals_full_geometry_autograd(kind):
    """rune tests/test_mobius_equivariant.py:111-121 / :214-232 (rtol 2e-7)."""
    p, w = _small(kind)
    s = _cell()
    pos, r, a = _edges(s, p)
    types = torch.tensor([0, 1, 0, 1])
    out = OM.forward(w, p, pos, types, [4], r, a)
    ref = OM.geometry_forward(w, p, pos, types, [4], r, a)
    for k in ("energy", "forces", "virial"):
        torch.testing.assert_close(out[k], ref[k], rtol=2e-7, atol=2e-8)


@pytest.mark.parametrize("kind", ["local", "eq"])
def test_forces_and_virial_match_finite_differences(kind):
    """rune tests/test_mobius_equivariant.py:184-211 (step 2e-5)."""
    p, w = _small(kind)
    s = _cell()
    pos, r, a = _edges(s, p)
    types = torch.tensor([0, 1, 0, 1])
    out = OM.forward(w, p, pos, types, [4], r, a)

    def energy(pp, rr, aa):
        return OM.forward(w, p, pp, types, [4], rr, aa, compute_forces=False,
                          compute_virial=False)["energy"].item()

    h = 2e-5
    fd = torch.zeros_like(pos)
    for i in range(4):
        for c in range(3):
            d = torch.zeros_like(pos)
            d[i, c] = h
            fd[i, c] = -(energy(pos + d, r, a) - energy(pos - d, r, a)) / (2 * h)
    torch.testing.assert_close(out["forces"], fd, rtol=2e-5, atol=3e-7)
    vfd = torch.zeros(3, 3, dtype=torch.float64)
    for i in range(3):
        for j in range(3):
            e = torch.zeros(3, 3, dtype=torch.float64)
            e[i, j] = h
            vals = []
            for sgn in (1, -1):
                m = torch.eye(3, dtype=torch.float64) + sgn * e
                rr = OM.Edges(r.center, r.neighbor, r.offsets @ m.T)
                aa = OM.Edges(a.center, a.neighbor, a.offsets @ m.T)
                vals.append(energy(pos @ m.T, rr, aa))
            vfd[i, j] = -(vals[0] - vals[1]) / (2 * h)
    torch.testing.assert_close(out["virial"].reshape(3, 3), vfd, rtol=2e-5, atol=3e-7)


@pytest.mark.parametrize("parity", [1, -1])
def test_rotation_and_reflection(parity):
    """rune tests/test_mobius_equivariant.py:152-181."""
    p, w = _small("eq")
    s = _cell()
    axis = np.array([1.0, -2.0, 3.0]) / math.sqrt(14.0)
    K = np.array([[0, -axis[2], axis[1]], [axis[2], 0, -axis[0]], [-axis[1], axis[0], 0]])
    R = (np.eye(3) + math.sin(0.713) * K + (1 - math.cos(0.713)) * K @ K) * parity
    types = torch.tensor([0, 1, 0, 1])
    pos, r, a = _edges(s, p)
    out = OM.forward(w, p, pos, types, [4], r, a)
    pos2, r2, a2 = _edges(s, p, R)
    rot = OM.forward(w, p, pos2, types, [4], r2, a2)
    Rt = torch.as_tensor(R)
    torch.testing.assert_close(rot["energy"], out["energy"], rtol=3e-6, atol=3e-7)
    torch.testing.assert_close(rot["forces"], out["forces"] @ Rt.T, rtol=3e-6, atol=3e-7)
    torch.testing.assert_close(rot["virial"].reshape(3, 3),
                               Rt @ out["virial"].reshape(3, 3) @ Rt.T, rtol=3e-6, atol=3e-7)
    torch.testing.assert_close(out["forces"].sum(0), torch.zeros(3, dtype=torch.float64),
                               rtol=0, atol=2e-10)


def test_nep_oracle_contraction_equals_geometry_autograd():
    from rune_amd.nep.model import seeded_nep
    model = seeded_nep(seed=5, elements=("Fe", "C"), rcut=(4.8, 4.0), max_neighbors=(500, 500))
    with torch.no_grad():
        model.q_scaler.uniform_(0.2, 0.5)
    p = model.params
    w = {k: v.double() for k, v in model.state_dict().items()}
    s = _cell()
    pos, r, a = _edges(s, p)
    types = torch.tensor([0, 1, 0, 1])
    out = OM.nep_forward(w, p, pos, types, [4], r, a)
    ref = OM.geometry_forward(w, p, pos, types, [4], r, a, energy_fn=OM.nep_geometry_energies)
    for k in ("energy", "forces", "virial"):
        torch.testing.assert_close(out[k], ref[k], rtol=2e-7, atol=2e-8)


def test_empty_neighbours_give_zero_forces():
    """rune tests/test_mobius_equivariant.py:322-333 (no edges)."""
    p, w = _small("eq")
    s = W.Structure(np.array([[1.0, 1, 1], [15.0, 15, 15]]), np.array([26, 6]), np.eye(3) * 30)
    pos, r, a = _edges(s, p)
    assert r.center.numel() == 0
    out = OM.forward(w, p, pos, torch.tensor([0, 1]), [2], r, a)
    assert torch.count_nonzero(out["forces"]) == 0
    assert torch.count_nonzero(out["virial"]) == 0
