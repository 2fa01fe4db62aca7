"""The ASE calculator and batch builder (rune/mobius/interface/calculator.py:
42-85, batch.py:124-166; the NEP ones are the same) on the HIP evaluator.

Cases of rune/tests/test_calculators.py:30-86 plus the stress convention:
energy and forces against the fp64 oracle, stress = Voigt(-W / V) in the
order [xx, yy, zz, yz, xz, xy] on a sheared triclinic cell,
PropertyNotImplementedError with stress disabled, ValueError for a
non-positive volume and for unsupported elements, fp64 periodic offsets, and
BatchBuilder.build against the oracle's padding (batch.py:9-39).  ASE runs
as the test-only stand-in of tests/ase_standin when it is not installed.
Needs an MI355X; run with ``-m gpu``.
"""

from importlib import import_module

import numpy as np
import pytest
import torch
from ase import Atoms
from ase.calculators.calculator import PropertyNotImplementedError

from oracle import model as OM
from oracle import neighbors as ONB

pytestmark = pytest.mark.gpu


def small_model(name, *, equivariant=False):
    """``small_model`` of rune/tests/test_calculators.py:12-26."""
    plugin = import_module(f"rune_amd.{name}.plugin")
    values = dict(elements=["H"], rcut_radial=3.5, rcut_angular=3.4, n_max_radial=1,
                  n_max_angular=1, basis_size_radial=1, basis_size_angular=1, l_max=2,
                  l_max_4body=0)
    if name == "nep":
        values["hidden_dims"] = [4]
    else:
        values.update(hidden_dim=8, ffn_dim=12, blocks=1, message_layers=1, message_dim=4,
                      pair_dim=2, message_groups=2, vector_channels=2)
        if equivariant:
            values.update(message_mode="equivariant", equivariant_channels=2)
    torch.manual_seed(3)
    return plugin, plugin.build_model(plugin.resolve_params(values))


def _save(plugin, model, path):
    torch.save(dict(plugin={"name": plugin.PLUGIN_NAME}, model_params=model.params,
                    model_state_dict=model.state_dict()), path)
    return path


def _oracle64(model, atoms):
    p = model.params
    w = {k: v.double() if v.is_floating_point() else v for k, v in model.state_dict().items()}
    nl = ONB.build(atoms.positions, atoms.cell.array, atoms.pbc, p["rcut_radial"],
                   p["rcut_angular"])
    sp = ONB.split(nl)
    mk = lambda k: OM.Edges(torch.as_tensor(sp[k][0]), torch.as_tensor(sp[k][1]),
                            torch.as_tensor(sp[k][2]))
    types = torch.tensor([p["elements"].index(
        __import__("ase").data.chemical_symbols[int(z)]) for z in atoms.numbers])
    fwd = OM.nep_forward if model.model_family == "nep" else OM.forward
    return fwd(w, p, torch.as_tensor(atoms.positions), types, [len(atoms)], mk("radial"),
               mk("angular"))


@pytest.mark.parametrize("name,equivariant", [("nep", False), ("mobius", False),
                                              ("mobius", True)])
def test_checkpoint_loader_and_calculator_results(name, equivariant, tmp_path):
    plugin, model = small_model(name, equivariant=equivariant)
    model = model.double().eval()
    with torch.no_grad():
        for parameter in model.parameters():
            parameter.add_(1.23456789e-9)
    artifact = _save(plugin, model, tmp_path / "model.pt")
    restored = plugin.load_model(artifact, device="cpu").eval()
    for key, expected in model.state_dict().items():
        torch.testing.assert_close(restored.state_dict()[key], expected, rtol=0, atol=0)
    calculator = plugin.build_calculator(artifact)     # reference default device="cpu"
    atoms = Atoms("H2", positions=[[0, 0, 0], [0.9, 0.1, 0]], cell=[8, 8, 8])
    batch = calculator._build_batch(atoms, compute_forces=True, compute_virial=True)
    assert batch["positions"].device.type == "cpu" and batch["positions"].dtype == torch.float64
    with torch.no_grad():
        expected = model(batch)
    calculator.calculate(atoms, ["energy", "forces", "stress"])
    res = calculator.results
    assert isinstance(res["energy"], float) and res["free_energy"] == res["energy"]
    # the padded batch and the calculator's own lists hold the same edges
    assert abs(res["energy"] - float(expected["energy"][0])) <= 1e-6
    np.testing.assert_allclose(res["forces"], expected["forces"].numpy(), rtol=0, atol=1e-5)
    stress = -expected["virial"][0].numpy().reshape(3, 3) / atoms.get_volume()
    np.testing.assert_allclose(res["stress"][:3], np.diag(stress), rtol=0, atol=1e-7)
    ref = _oracle64(model, atoms)
    assert abs(res["energy"] - float(ref["energy"][0])) <= 1e-5 * len(atoms)
    np.testing.assert_allclose(res["forces"], ref["forces"].numpy(), rtol=0, atol=1e-4)


def test_double_precision_periodic_offsets_are_not_rounded_to_float32():
    spacing = 3.1234567890123
    atoms = Atoms("H", positions=[[0.1, 0.2, 0.3]], cell=[spacing, 4.2, 5.3], pbc=True)
    for name in ("nep", "mobius"):
        _, model = small_model(name)
        builder_type = import_module(f"rune_amd.{name}.interface.batch").BatchBuilder
        batch = builder_type(model.params, torch.device("cpu"), torch.float64).build(
            atoms, compute_forces=True, compute_virial=True)
        for kind in ("radial", "angular"):
            offsets = batch[f"{kind}_offsets"][batch[f"{kind}_neighbors"] >= 0]
            assert sorted(offsets[:, 0].tolist()) == [-spacing, spacing]


def test_ase_stress_switch_and_unsupported_elements(tmp_path):
    for name in ("nep", "mobius"):
        plugin, model = small_model(name)
        artifact = _save(plugin, model, tmp_path / f"{name}.pt")
        atoms = Atoms("H2", positions=[[0, 0, 0], [0.9, 0, 0]], cell=[8, 8, 8])
        atoms.calc = plugin.build_calculator(artifact, compute_stress=False)
        assert np.isfinite(atoms.get_potential_energy())
        assert atoms.get_forces().shape == (2, 3)
        with pytest.raises(PropertyNotImplementedError):
            atoms.get_stress()
        kind = "NEP" if name == "nep" else "Möbius"
        atoms[0].symbol = "He"
        with pytest.raises(ValueError, match=f"not supported by this {kind} model"):
            atoms.get_potential_energy()


def test_stress_sign_and_voigt_order_on_a_sheared_cell():
    """stress = full_3x3_to_voigt_6_stress(-W / V) with W_ab = -sum_e g_a r_b
    (calculator.py:83-85): every Voigt component against the fp64 oracle."""
    from rune_amd import MODELS
    from rune_amd.mobius import plugin
    calc = plugin.build_calculator(MODELS["mobius-oam-loc"])
    cell = np.array([[5.43, 0.35, -0.2], [0.15, 5.5, 0.4], [-0.3, 0.25, 5.6]])
    rng = np.random.default_rng(12)
    frac = np.array([[0, 0, 0], [.5, .5, 0], [.5, 0, .5], [0, .5, .5],
                     [.25, .25, .25], [.75, .75, .25], [.75, .25, .75], [.25, .75, .75]])
    atoms = Atoms("Si8", scaled_positions=frac + rng.normal(0, 0.01, (8, 3)), cell=cell,
                  pbc=True)
    atoms.calc = calc
    got = atoms.get_stress()
    ref = _oracle64(calc.model, atoms)
    w = ref["virial"][0].numpy().reshape(3, 3)
    s = -w / atoms.get_volume()
    expect = np.array([s[0, 0], s[1, 1], s[2, 2], 0.5 * (s[1, 2] + s[2, 1]),
                       0.5 * (s[0, 2] + s[2, 0]), 0.5 * (s[0, 1] + s[1, 0])])
    assert abs(s[1, 2]) > 1e-4 and abs(s[0, 2]) > 1e-4 and abs(s[0, 1]) > 1e-4
    np.testing.assert_allclose(got, expect, rtol=0, atol=1e-5 * 8 / atoms.get_volume())
    np.testing.assert_allclose(atoms.get_forces(), ref["forces"].numpy(), rtol=0, atol=1e-4)


def test_non_positive_volume_is_rejected(tmp_path):
    plugin, model = small_model("mobius")
    artifact = _save(plugin, model, tmp_path / "m.pt")
    calc = plugin.build_calculator(artifact)
    atoms = Atoms("H2", positions=[[0, 0, 0], [0.9, 0, 0]], cell=[0, 0, 0])
    with pytest.raises(ValueError, match="positive cell volume"):
        calc.calculate(atoms, ["energy", "stress"])
    calc.calculate(atoms, ["energy", "forces"])      # a cluster without stress is fine
    assert calc.results["forces"].shape == (2, 3)


def test_batch_builder_matches_reference_padding():
    """BatchBuilder.build against the oracle's list packed as batch.py:9-39."""
    from rune_amd import MODELS
    from rune_amd.mobius import plugin
    from rune_amd.mobius.interface.batch import BatchBuilder
    model = plugin.load_model(MODELS["mobius-oam-mp"])
    p = model.params
    rng = np.random.default_rng(4)
    cell = np.diag([7.1, 7.3, 6.9]) + rng.uniform(-0.3, 0.3, (3, 3))
    atoms = Atoms(numbers=rng.choice([26, 24, 28], 24), positions=rng.random((24, 3)) @ cell,
                  cell=cell, pbc=True)
    batch = BatchBuilder(p, "cpu", torch.float32).build(atoms, compute_forces=True,
                                                        compute_virial=False)
    nl = ONB.build(atoms.positions, cell, atoms.pbc, p["rcut_radial"], p["rcut_angular"])
    sp = ONB.split(nl)
    for kind in ("radial", "angular"):
        nb, of = ONB.pack(*sp[kind], len(atoms), p[f"max_neighbors_{kind}"])
        np.testing.assert_array_equal(batch[f"{kind}_neighbors"].numpy(), nb)
        np.testing.assert_array_equal(batch[f"{kind}_offsets"].numpy(), of.astype(np.float32))
    assert batch["compute_forces"] is True and batch["compute_virial"] is False
    assert batch["types"].tolist() == [p["elements"].index({26: "Fe", 24: "Cr", 28: "Ni"}[z])
                                       for z in atoms.numbers]
