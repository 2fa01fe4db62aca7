"""mobius.txt / nep.txt formats, checkpoint loading and parameter validation (CPU)."""

import math

import numpy as np
import pytest
import torch

from oracle import model as OM
from rune_amd import MODELS
from rune_amd.mobius import export as EX
from rune_amd.mobius import plugin as MP
from rune_amd.nep import plugin as NP
from tests.golden.make_golden import EXPORT_CASES, small_export_model
from tests.helpers import GOLDEN


@pytest.mark.parametrize("kind", list(EXPORT_CASES))
def test_mobius_txt_matches_reference_exporter_bytes(kind, tmp_path):
    """Same bytes as rune/mobius/export.py on the same model (fixture from the reference)."""
    model = small_export_model(kind)
    path = MP.export_model(model, tmp_path / "model")
    assert path.name == "mobius.txt"
    assert path.read_text() == (GOLDEN / f"export_{kind}.mobius.txt").read_text()


@pytest.mark.parametrize("name", ["mobius-oam-loc", "mobius-oam-eq"])
def test_mobius_txt_preserves_weights_bitwise(name, tmp_path):
    model = MP.load_model(MODELS[name])
    # a reduced copy keeps the file small: same code path, 89-type tables
    path = EX.export_model(model, tmp_path / "model_epoch_3")
    assert path.name == "mobius_epoch_3.txt"
    elements, ints, reals, tensors = EX.read_mobius_txt(path)
    assert elements == model.elements
    assert ints["num_L"] == 10 and ints["input_dim"] == 103
    for key, value in model.state_dict().items():
        assert torch.equal(tensors[key], value.double()), key


def test_exported_basis_table_evaluates_to_angular_basis():
    """rune tests/test_mobius_export.py:76-96: sparse polynomials == _compute_basis."""
    model = small_export_model("eq")
    rows, offsets = EX.angular_polynomials(model.descriptor.angular)
    rng = np.random.default_rng(0)
    u = rng.normal(size=(50, 3))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    ut = torch.as_tensor(u)
    Z = OM.z_tables({f"descriptor.angular.Z{L}": getattr(model.descriptor.angular, f"Z{L}")
                     for L in range(1, 9)}, torch.float64)
    ref = OM.angular_basis(ut, 4, Z).numpy()
    got = np.zeros_like(ref)
    for comp, coef, xp, yp, zp in rows.tolist():
        got[:, int(comp)] += coef * u[:, 0] ** xp * u[:, 1] ** yp * u[:, 2] ** zp
    np.testing.assert_allclose(got, ref, rtol=2e-12, atol=1e-13)
    assert offsets[-1] == len(rows)


def test_exported_invariant_table_evaluates_to_invariants():
    """rune tests/test_mobius_export.py:98-122: sparse invariants == _compute_q."""
    model = small_export_model("eq")
    ang = model.descriptor.angular
    rows, offsets = EX.invariant_polynomials(ang)
    s = torch.randn(7, 2, 24, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    flags = OM.Flags(4, 1, 1, 1, 1, 1, 1)
    w = {f"descriptor.angular.{k}": getattr(ang, k) for k in ("C3B", "C4B", "C5B", "C4B2")}
    ref = OM.invariants(s, flags, w).numpy()
    got = np.zeros_like(ref)
    sn = s.numpy()
    for out, coef, deg, *idx in rows.tolist():
        term = np.ones(sn.shape[:2])
        for k in idx[:int(deg)]:
            term = term * sn[..., int(k)]
        got[..., int(out)] += coef * term
    np.testing.assert_allclose(got, ref, rtol=2e-12, atol=1e-13)


def test_export_rejects_nonfinite(tmp_path):
    model = small_export_model("local")
    with torch.no_grad():
        model.input_projection.weight[0, 0] = float("nan")
    with pytest.raises(ValueError, match="nonfinite"):
        EX.export_model(model, tmp_path / "model")


def test_checkpoints_load_strict_and_keep_float32():
    for name, path in MODELS.items():
        model = MP.load_model(path)
        ck = torch.load(path, weights_only=True)
        assert list(model.state_dict().keys()) == list(ck["model_state_dict"].keys())
        for k, v in ck["model_state_dict"].items():
            assert torch.equal(model.state_dict()[k], v), k
        assert next(model.parameters()).dtype == torch.float32


def test_nep_txt_roundtrip(tmp_path):
    from rune_amd.nep.model import seeded_nep
    model = seeded_nep(seed=3)
    with torch.no_grad():
        model.q_scaler.uniform_(0.5, 2.0)
        model.shared_bias.fill_(0.125)
    path = NP.export_model(model, tmp_path / "model")
    assert path.name == "nep.txt"
    back = NP.load_model(path)
    for k, v in model.state_dict().items():
        torch.testing.assert_close(back.state_dict()[k], v, rtol=1e-9, atol=1e-10, msg=k)
    lines = path.read_text().splitlines()
    assert lines[0] == "nep4 2 Pb Te"
    assert lines[1] == "cutoff 6.0 4.0 100 30"
    assert lines[4] == "l_max 4 2 0"        # zeros trimmed only beyond 3 entries
    assert lines[5] == "ANN 30 0"
    assert lines[6] == f"{model.element_mlps['Pb'][0].weight[0, 0].item():18.10e}"


def test_nep_txt_rejects_unsupported(tmp_path):
    p = tmp_path / "bad.txt"
    p.write_text("nep5 1 H\n")
    with pytest.raises(NotImplementedError):
        NP.load_model(p)
    p.write_text("nep4 1 H\ncutoff 5 4 10 10\nn_max 1 1\nbasis_size 1 1\nl_max 4\nANN 4 1\n")
    with pytest.raises(ValueError, match="single-hidden-layer"):
        NP.load_model(p)


@pytest.mark.parametrize("changes,field", [
    ({"message_mode": "unknown"}, "message_mode"),
    ({"message_layers": 0}, "message_layers"),
    ({"equivariant_channels": 0}, "equivariant_channels"),
    ({"equivariant_channels": True}, "equivariant_channels"),
    ({"equivariant_l_max": 0}, "equivariant_l_max"),
    ({"equivariant_l_max": 5}, "equivariant_l_max"),
    ({"equivariant_l_max": 1.5}, "equivariant_l_max"),
    ({"l_max": 9, "equivariant_l_max": 8}, "l_max"),
])
def test_mobius_parameter_validation(changes, field):
    """Cases of rune tests/test_mobius_equivariant.py:442-458."""
    values = {"elements": ["Fe", "C"], "message_mode": "equivariant", "message_layers": 2,
              "equivariant_channels": 3, "l_max": 4}
    values.update(changes)
    with pytest.raises(ValueError, match=field):
        MP.resolve_params(values)


def test_direction_order_defaults_to_descriptor_order():
    p = MP.resolve_params({"elements": ["H"], "message_mode": "equivariant", "l_max": 3})
    assert p["equivariant_l_max"] == 3


def test_nep_parameter_limits():
    with pytest.raises(ValueError, match="n_max_radial"):
        NP.resolve_params({"elements": ["H"], "n_max_radial": 13})
    with pytest.raises(ValueError, match="cutoffs"):
        NP.resolve_params({"elements": ["H"], "rcut_radial": 5.0, "rcut_angular": 6.0})
    with pytest.raises(ValueError, match="Unknown model parameter"):
        NP.resolve_params({"elements": ["H"], "bogus": 1})


def test_calculator_requires_device(monkeypatch):
    from rune_amd import _native as N
    with pytest.raises(RuntimeError, match="HIP"):
        N.require_device("cpu")
