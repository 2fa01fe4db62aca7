"""The reference's own native-evaluator cases, HIP path against the CPU oracle.

``rune/tests/test_mobius_gpumd.py`` checks the reference's GPUMD evaluator
against the Python model on a fixed set of structures and model options
(small triclinic cell with self-images, large cell, empty edges, angular
cutoff above the radial one with ZBL, non-warp-aligned widths, descriptor
orders 1/2/6/8, mixed PBC, flexible ZBL, positions several periods outside
the cell, changing and empty neighbourhoods over a trajectory, neighbour
capacity).  The same cases run here through the C ABI (``Evaluator`` ->
``torch.ops.rune_hip.evaluate`` / ``rune_model_compute``) and are compared
with the fp64 oracle: per-atom energies, forces, the structure virial and the
per-atom virial attributed to the neighbour atom (``rune/mobius/model.py:
23-44``), within the fp32 tolerances 1e-5 eV, 1e-4 eV/Å and 1e-5 eV/atom
(per-atom virial components: 1e-4 eV).  The reference fp32 path (the oracle
in fp32) is printed beside it, and the HIP result is also compared with it.
Needs an MI355X; run with ``-m gpu``.
"""

import numpy as np
import pytest
import torch

from oracle import model as OM
from oracle import neighbors as ONB
from rune_amd import workloads as W

pytestmark = pytest.mark.gpu

TOL_E, TOL_F, TOL_W, TOL_WA = 1e-5, 1e-4, 1e-5, 1e-4


def model_for(mode, **changes):
    """``model_for`` of rune/tests/test_mobius_gpumd.py:34-50 (fp32 weights)."""
    from rune_amd.mobius.model import Mobius
    from rune_amd.mobius.plugin import resolve_params
    config = dict(elements=["Fe", "C"], hidden_dim=8, ffn_dim=12, blocks=1,
                  message_layers=0 if mode == "local" else 2, message_dim=8,
                  message_groups=2, pair_dim=3, vector_channels=2,
                  message_basis_size=3, rcut_radial=3.8, rcut_angular=3.5,
                  n_max_radial=1, n_max_angular=1,
                  basis_size_radial=2, basis_size_angular=2,
                  l_max=4, l_max_4body=2, l_max_5body=1,
                  has_q_112=1, has_q_123=1, has_q_233=1, has_q_134=1,
                  max_neighbors_radial=128, max_neighbors_angular=128)
    if mode == "equivariant":
        config.update(message_mode="equivariant", equivariant_channels=3,
                      equivariant_l_max=4)
    config.update(changes)
    torch.manual_seed(20261021)
    model = Mobius(resolve_params(config)).eval()
    with torch.no_grad():
        model.q_scaler.copy_(torch.linspace(.7, 1.2, model.q_scaler.numel()))
    return model


def small_atoms(pbc=(True, True, True)):
    cell = np.array([[4.1, .1, .2], [.0, 4.3, .1], [.1, .0, 4.5]])
    frac = np.array([[.10, .13, .22], [.82, .21, .37], [.30, .75, .19], [.68, .63, .81]])
    return W.Structure(frac @ cell, np.array([26, 6, 26, 6]), cell, pbc=tuple(pbc))


def large_atoms(pbc=(True, True, True)):
    pos = np.array([[.2, .3, .4], [19.2, .6, .4], [2., 1., .7], [8., 7., 9.], [9.8, 7.2, 8.1],
                    [14., 14., 14.]])
    cell = np.array([[20., .2, .4], [0., 20.5, .3], [.2, 0., 21.]])
    return W.Structure(pos, np.array([26, 6, 26, 6, 26, 6]), cell, pbc=tuple(pbc))


def _oracle(model, s, types, dtype):
    p = model.params
    sd = model.state_dict()
    w = {k: v.to(dtype) if v.is_floating_point() else v for k, v in sd.items()}
    nl = ONB.build(s.positions, s.cell, s.pbc, p["rcut_radial"], p["rcut_angular"])
    sp = ONB.split(nl)
    mk = lambda k: OM.Edges(torch.as_tensor(sp[k][0]), torch.as_tensor(sp[k][1]),
                            torch.as_tensor(sp[k][2], dtype=dtype))
    fwd = OM.nep_forward if model.model_family == "nep" else OM.forward
    return fwd(w, p, torch.as_tensor(s.positions, dtype=dtype),
               torch.as_tensor(types, dtype=torch.long), [len(s)], mk("radial"), mk("angular"))


def _diff(out, ref, n):
    g = lambda k: out[k].detach().cpu().double().numpy()
    r = lambda k: ref[k].detach().double().numpy()
    return (np.abs(g("energies") - r("energies")).max(initial=0.0),
            np.abs(g("forces") - r("forces")).max(initial=0.0),
            np.abs(g("virial")[0] - r("virial")[0]).max() / max(n, 1),
            np.abs(g("atom_virial") - r("atom_virial")).max(initial=0.0))


def check(model, s, label="", ev=None):
    """HIP vs fp64 oracle (bar: the stated tolerances, or 2x the reference
    fp32 path's own deviation where that is larger), and HIP vs the fp32
    oracle, on E_i, F, W and the per-atom virial."""
    from rune_amd import _native as N
    from rune_amd.api import Evaluator
    if ev is None:
        family = N.FAMILY_NEP if model.model_family == "nep" else N.FAMILY_MOBIUS
        ev = Evaluator(model.params, model.state_dict(), family)
    types = ev.types_of(s.numbers)
    out = ev.evaluate(s, atom_virial=True)
    return compare(model, s, types, out, label)


def compare(model, s, types, out, label):
    r64 = _oracle(model, s, types, torch.float64)
    r32 = _oracle(model, s, types, torch.float32)
    hip = _diff(out, r64, len(s))
    ref = _diff(r32, r64, len(s))
    vs32 = _diff(out, r32, len(s))
    print(f"{label}: HIP-fp64 {['%.1e' % x for x in hip]}  ref32-fp64 "
          f"{['%.1e' % x for x in ref]}  HIP-ref32 {['%.1e' % x for x in vs32]}")
    for h, r, v, t in zip(hip, ref, vs32, (TOL_E, TOL_F, TOL_W, TOL_WA)):
        assert h <= max(t, 2.0 * r), (label, hip, ref)
        # against the reference fp32 path: the stated tolerance, widened only
        # by that path's own distance from exact arithmetic
        assert v <= t + r, (label, vs32, ref)
    return out


@pytest.mark.parametrize("mode", ["local", "scalar", "equivariant"])
def test_three_modes_triclinic_periodic_images(mode):
    check(model_for(mode), small_atoms(), f"{mode}-small")


@pytest.mark.parametrize("mode", ["local", "scalar", "equivariant"])
def test_three_modes_large_cell(mode):
    check(model_for(mode), large_atoms(), f"{mode}-large")


@pytest.mark.parametrize("mode", ["local", "scalar", "equivariant"])
def test_empty_edges_and_runtime_model_dimensions(mode):
    s = W.Structure(np.array([[2., 2., 2.], [12., 12., 12.]]), np.array([26, 6]),
                    np.eye(3) * 30.0)
    model = model_for(mode, hidden_dim=16, ffn_dim=24, message_dim=12, blocks=2,
                      activation="tanh")
    out = check(model, s, f"{mode}-empty")
    assert torch.count_nonzero(out["forces"]) == 0


def test_angular_cutoff_above_radial_and_zbl():
    model = model_for("equivariant", rcut_radial=3., rcut_angular=4.2, zbl=[.8, 2.8],
                      equivariant_l_max=2)
    check(model, small_atoms(), "angular-zbl")


@pytest.mark.parametrize("mode", ["local", "scalar", "equivariant"])
def test_non_warp_aligned_network_channels(mode):
    model = model_for(mode, hidden_dim=36, ffn_dim=53, message_dim=15, message_groups=3,
                      blocks=2)
    check(model, small_atoms(), f"{mode}-warp-tail")


@pytest.mark.parametrize("order", [1, 2, 6, 8])
def test_descriptor_derivatives_across_angular_orders(order):
    model = model_for("equivariant", l_max=order, equivariant_l_max=min(order, 3),
                      l_max_4body=2 if order >= 2 else 0, has_q_112=int(order >= 2),
                      has_q_123=int(order >= 3), has_q_233=int(order >= 3),
                      has_q_134=int(order >= 4))
    check(model, small_atoms(), f"order-{order}")


@pytest.mark.parametrize("channels", [2, 3, 5, 17, 33])
def test_radial_channels_and_basis_group_boundaries(channels):
    """Channel counts past 16 and long bases run the descriptor kernels that
    keep per-lane rows in LDS."""
    model = model_for("local", n_max_radial=channels - 1, n_max_angular=channels - 1,
                      basis_size_radial=20, basis_size_angular=18)
    check(model, small_atoms(), f"channels-{channels}")


@pytest.mark.parametrize("mode", ["scalar", "equivariant"])
def test_wide_descriptor_with_message_blocks(mode):
    """17 radial / 19 angular channels and 30 / 26 basis functions feeding MP
    and EQ blocks (the direction encoder projects 19 angular channels)."""
    model = model_for(mode, n_max_radial=16, n_max_angular=18, basis_size_radial=29,
                      basis_size_angular=25)
    check(model, small_atoms(), f"{mode}-wide-descriptor")


def test_equivariant_order_eight():
    """equivariant_l_max = 8, the reference's largest (rune/mobius/plugin.py:81-86)."""
    model = model_for("equivariant", l_max=8, equivariant_l_max=8)
    check(model, small_atoms(), "eq-order-8")
    check(model, large_atoms(), "eq-order-8-large")


def test_mixed_pbc_and_additional_model_options():
    check(model_for("local", activation="gelu"), small_atoms((True, False, True)),
          "mixed-small-gelu")
    check(model_for("scalar", vector_channels=0), large_atoms((True, False, True)),
          "mixed-large-vector0")
    coefficients = [.18175, 3.1998, .50986, .94229, .28022, .4029, .02817, .20162]
    zbl = dict(rc_inner=0., rc_outer=0., flexible=True, parameters=[[.5, 2.8, *coefficients]] * 3)
    check(model_for("equivariant", zbl=zbl), small_atoms((True, False, True)), "flexible-zbl")


def test_flexible_zbl_distinct_pair_rows():
    """Three elements with six distinct flexible rows: the row of each type pair."""
    rows = []
    for r in range(6):
        co = []
        for k in range(4):
            co += [0.1 * (k + 1) + 0.01 * r, 0.5 * (k + 1) + 0.02 * r]
        rows.append([0.4 + 0.05 * r, 2.6 + 0.05 * r] + co)
    zbl = dict(rc_inner=0., rc_outer=0., flexible=True, parameters=rows)
    model = model_for("local", elements=["Fe", "C", "O"], zbl=zbl)
    rng = np.random.default_rng(7)
    cell = np.diag([7.0, 7.2, 7.4])
    s = W.Structure(rng.random((10, 3)) @ cell, rng.choice([26, 6, 8], 10), cell)
    check(model, s, "flexible-zbl-rows")


def test_positions_outside_multiple_periods():
    s = W.Structure(np.array([[1., 1., 1.], [64.7, 1., 1.], [8., 8., 8.], [-55.8, 8., 8.]]),
                    np.array([26, 6, 26, 6]), np.eye(3) * 20.9)
    check(model_for("equivariant"), s, "unwrapped-large")


def test_neighbor_capacity_is_rejected():
    from rune_amd import _native as N
    from rune_amd.api import Evaluator
    model = model_for("local", max_neighbors_radial=1)
    ev = Evaluator(model.params, model.state_dict(), N.FAMILY_MOBIUS)
    with pytest.raises(ValueError, match="exceeds max_neighbors=1"):
        ev.evaluate(small_atoms())


@pytest.mark.parametrize("mode", ["local", "scalar", "equivariant"])
def test_workspace_reuse_with_changing_and_empty_neighbors(mode):
    """A fast atom passes two separated atoms, then leaves both cutoffs: 0 -> 2
    -> 4 -> 2 -> 0 directed edges in one evaluator, every frame against the
    oracle (retained workspace must not leak into later frames)."""
    from rune_amd import _native as N
    from rune_amd.api import Evaluator
    model = model_for(mode, blocks=2)
    ev = Evaluator(model.params, model.state_dict(), N.FAMILY_MOBIUS)
    counts = []
    for k in range(13):
        x = 25.0 - 1.2 * k
        s = W.Structure(np.array([[15., 15., 15.], [20., 15., 15.], [x, 16.3, 15.]]),
                        np.array([26, 6, 26]), np.eye(3) * 40.0)
        nl = ONB.build(s.positions, s.cell, s.pbc, model.params["rcut_radial"],
                       model.params["rcut_angular"])
        counts.append(int(nl["radial_mask"].sum()))
        check(model, s, f"{mode}-frame-{k}", ev)
    assert counts[0] == 0 and max(counts) >= 4 and counts[-1] == 0


@pytest.mark.parametrize("mode", ["local", "scalar", "equivariant"])
def test_neighbors_enter_cutoff_within_skin_displacement(mode):
    """Skin reuse (rune_nlist_update, 1 Å skin) with the oracle in the loop: a
    pair starts outside the cutoff but inside the skin and moves into it by
    less than skin / 2, so the cached candidates must produce the new edges."""
    from rune_amd import _native as N
    model = model_for(mode)
    p = model.params
    native = N.NativeModel(p, model.state_dict(), N.FAMILY_MOBIUS)
    nl = N.NeighborList()
    searched, counts = [], []
    cell = np.eye(3) * 40.0
    for k in range(12):
        sep = 4.2 - 0.04 * k      # 0.44 Å in all: below skin / 2, into rc = 3.8
        s = W.Structure(np.array([[15., 15., 15.], [15. + sep, 15., 15.]]),
                        np.array([26, 6]), cell)
        pos = torch.as_tensor(s.positions, device="cuda")
        searched.append(nl.update(pos, [0, 2], [cell], [np.ones(3, np.int32)],
                                  p["rcut_radial"], p["rcut_angular"], p["max_neighbors_radial"],
                                  p["max_neighbors_angular"], 1.0))
        types = torch.tensor([0, 1], dtype=torch.int32, device="cuda")
        out = native.compute(nl, types, 1, True, True, atom_virial=True)
        counts.append(nl.n_records)
        compare(model, s, [0, 1], out, f"{mode}-skin-step-{k}")
    assert searched[0] and not any(searched[1:])
    assert counts[0] == 0 and counts[-1] == 2


def test_empty_structure_gives_zero_energy_and_virial():
    from rune_amd import _native as N
    from rune_amd.api import Evaluator
    model = model_for("local")
    ev = Evaluator(model.params, model.state_dict(), N.FAMILY_MOBIUS)
    s = W.Structure(np.zeros((0, 3)), np.zeros(0, np.int64), np.eye(3) * 10.0)
    for _ in range(2):    # the second call reuses a workspace that held other values
        ev.evaluate(small_atoms())
        out = ev.evaluate(s)
        assert out["energies"].numel() == 0 and out["forces"].shape == (0, 3)
        assert torch.count_nonzero(out["energy"]) == 0
        assert torch.count_nonzero(out["virial"]) == 0


# ---- NEP ----

def _nep(zbl=None, seed=11):
    from rune_amd.nep.model import NEP
    from rune_amd.nep.plugin import resolve_params
    values = {"elements": ["Pb", "Te"], "n_max_radial": 4, "n_max_angular": 4,
              "basis_size_radial": 8, "basis_size_angular": 8, "l_max": 4, "l_max_4body": 2,
              "l_max_5body": 0, "rcut_radial": 6.0, "rcut_angular": 4.0, "hidden_dims": [30],
              "max_neighbors_radial": 100, "max_neighbors_angular": 30}
    if zbl is not None:
        values["zbl"] = zbl
    torch.manual_seed(seed)
    model = NEP(resolve_params(values))
    with torch.no_grad():
        model.q_scaler.uniform_(0.5, 1.5)
    return model


def _compressed_rocksalt(seed):
    s = W.rocksalt(seed=seed, reps=2, a=5.2, sigma=0.15)
    return s


@pytest.mark.parametrize("kind", ["none", "universal", "flexible"])
def test_nep_zbl_on_the_angular_list(kind):
    """NEP ZBL pairs and the direct edge term use the angular list
    (rune/nep/model.py:93); a compressed cell puts pairs inside both tapers."""
    coefficients = [.18175, 3.1998, .50986, .94229, .28022, .4029, .02817, .20162]
    zbl = {"none": None, "universal": [1.5, 3.0],
           "flexible": dict(rc_inner=0., rc_outer=0., flexible=True,
                            parameters=[[1.2, 3.2, *coefficients], [1.4, 3.4, *coefficients],
                                        [1.6, 3.6, *coefficients]])}[kind]
    model = _nep(zbl)
    check(model, _compressed_rocksalt(60), f"nep-zbl-{kind}")


def test_nep_isolated_atoms_closed_form(tmp_path):
    """q = 0 without neighbours: E = sum_h w1 tanh(b0) - shared_bias exactly as
    the per-element network gives it (rune/nep/model.py:157-170)."""
    from rune_amd import _native as N
    from rune_amd.api import Evaluator
    model = _nep()
    with torch.no_grad():
        model.shared_bias.fill_(0.25)
    ev = Evaluator(model.params, model.state_dict(), N.FAMILY_NEP)
    s = W.Structure(np.array([[1., 1., 1.], [30., 1., 1.], [1., 30., 1.]]),
                    np.array([82, 52, 82]), np.zeros((3, 3)), pbc=(False, False, False))
    out = ev.evaluate(s, atom_virial=True)
    for a, el in enumerate(["Pb", "Te", "Pb"]):
        mlp = model.element_mlps[el]
        with torch.no_grad():
            expect = float((mlp[2].weight[0].double() * torch.tanh(mlp[0].bias.double())).sum()
                           - model.shared_bias.double())
        assert abs(out["energies"][a].item() - expect) <= 1e-6
    assert torch.count_nonzero(out["forces"]) == 0


# ---- neighbour builder: shifts beyond a few periods, cell-less clusters ----

def _records(s, rc_r, rc_a, limit=100000):
    from rune_amd import _native as N
    nl = N.NeighborList().build(torch.as_tensor(s.positions, device="cuda"), [0, len(s)],
                                [s.cell], [np.asarray(s.pbc, np.int32)], rc_r, rc_a, limit, limit)
    return nl, {k: v.cpu().numpy() for k, v in nl.export().items()}


def _assert_list_bit_exact(s, rc_r, rc_a, method="auto"):
    nl, out = _records(s, rc_r, rc_a)
    ref = ONB.build(s.positions, s.cell, s.pbc, rc_r, rc_a, method=method)
    assert nl.n_records == len(ref["neighbor"])
    np.testing.assert_array_equal(out["ptr"], ref["ptr"])
    np.testing.assert_array_equal(out["nbr"], ref["neighbor"])
    np.testing.assert_array_equal(out["shift"], ref["shift"])
    np.testing.assert_array_equal(out["vec"][:, :3], ref["vec32"])
    return nl


def test_atoms_hundreds_of_periods_apart_bit_exact():
    cell = np.array([[5.1, .2, 0.], [.1, 5.3, .2], [0., .3, 5.2]])
    frac = np.array([[.1, .2, .3], [200.6, .4, .5], [-150.3, 99.8, .1], [.7, -210.2, 180.9],
                     [.45, .55, .65]])
    s = W.Structure(frac @ cell, np.array([26, 6, 26, 6, 26]), cell)
    # the oracle's cell-list enumeration (brute force would visit 10^7 images)
    _assert_list_bit_exact(s, 4.5, 3.5, method="celllist")


def test_shift_beyond_range_is_an_error():
    cell = np.eye(3) * 5.0
    s = W.Structure(np.array([[1., 1., 1.], [1. + 5.0 * 600, 1., 1.]]), np.array([26, 6]), cell)
    with pytest.raises(ValueError, match="511 cell periods"):
        _records(s, 4.0, 3.0)


@pytest.mark.parametrize("n", [40, 3000])
def test_cell_less_cluster_bit_exact(n):
    rng = np.random.default_rng(n)
    side = (n / 0.08) ** (1 / 3)
    pos = rng.random((n, 3)) * side - 0.5 * side
    s = W.Structure(pos, np.full(n, 26), np.zeros((3, 3)), pbc=(False, False, False))
    _assert_list_bit_exact(s, 4.5, 3.5)


def test_cell_less_cluster_model_matches_oracle():
    rng = np.random.default_rng(3)
    pos = rng.random((30, 3)) * 7.0 - 20.0
    s = W.Structure(pos, rng.choice([26, 6], 30), np.zeros((3, 3)), pbc=(False, False, False))
    check(model_for("equivariant"), s, "cluster-eq")


def test_cell_less_cluster_search_scales_linearly():
    """A 64k-atom cluster in a zero cell: the bins cover its bounding box, so
    the search is far from an all-pairs O(N^2) scan (which would test 4e9
    pairs, hundreds of milliseconds)."""
    import time
    from rune_amd import _native as N
    n = 64000
    rng = np.random.default_rng(9)
    side = (n / 0.08) ** (1 / 3)
    pos = torch.as_tensor(rng.random((n, 3)) * side + 300.0, device="cuda")
    nl = N.NeighborList()
    args = ([0, n], [np.zeros((3, 3))], [np.zeros(3, np.int32)], 4.5, 3.5, 400, 400)
    nl.build(pos, *args)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(5):
        nl.build(pos, *args)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / 5 * 1e3
    print(f"64k-atom cluster search: {ms:.2f} ms, {nl.n_records} records")
    assert ms < 60.0
