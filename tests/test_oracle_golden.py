"""Pin the CPU oracle to the golden vectors recorded from the reference modules."""

import numpy as np
import pytest
import torch

from oracle import model as OM
from tests.helpers import edges_from, golden, load_weights

STRUCTS = ("fec4", "si8", "fcc32", "amo96")


def _cases():
    for m in ("loc", "mp", "eq"):
        for s in STRUCTS:
            if m != "loc" and s == "si8":
                continue
            yield m, s


@pytest.mark.parametrize("model,struct", list(_cases()))
def test_descriptor_and_contraction_match_reference(model, struct):
    p, w = load_weights(model)
    rec = golden(f"mobius_{model}_{struct}")
    pos = torch.as_tensor(rec["positions"])
    types = torch.as_tensor(rec["types"])
    r, a = edges_from(rec, "radial"), edges_from(rec, "angular")
    vr, va, s, q = OM._descriptor(w, p, pos, types, r, a)
    np.testing.assert_allclose(q.numpy(), rec["q"], rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(s.numpy(), rec["moments"], rtol=1e-11, atol=1e-12)
    f, v = OM.contract(w, p, pos, types, r, a, torch.as_tensor(rec["contract_dq"]),
                       torch.as_tensor(rec["contract_dmom"]))
    np.testing.assert_allclose(f.numpy(), rec["contract_forces"], rtol=1e-9, atol=1e-10)
    np.testing.assert_allclose(v.numpy(), rec["contract_atom_virial"], rtol=1e-9, atol=1e-10)


@pytest.mark.parametrize("model,struct", list(_cases()))
def test_energy_force_virial_match_reference_f64(model, struct):
    p, w = load_weights(model)
    rec = golden(f"mobius_{model}_{struct}")
    pos = torch.as_tensor(rec["positions"])
    types = torch.as_tensor(rec["types"])
    r, a = edges_from(rec, "radial"), edges_from(rec, "angular")
    out = OM.forward(w, p, pos, types, [len(pos)], r, a)
    np.testing.assert_allclose(out["energies"].numpy(), rec["energies_f64"], rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(out["forces"].numpy(), rec["forces_f64"], rtol=1e-8, atol=1e-9)
    np.testing.assert_allclose(out["virial"][0].numpy(), rec["virial_f64"], rtol=1e-8, atol=1e-8)


@pytest.mark.parametrize("model,struct", list(_cases()))
def test_energy_force_virial_match_reference_f32(model, struct):
    """fp32 oracle vs fp32 reference: the stated fp32 tolerances, or twice the
    reference fp32 path's own distance from its fp64 result where that is
    larger (fp32 sums on the CPU depend on the thread count)."""
    p, w = load_weights(model, torch.float32)
    rec = golden(f"mobius_{model}_{struct}")
    pos = torch.as_tensor(rec["positions"], dtype=torch.float32)
    types = torch.as_tensor(rec["types"])
    r, a = edges_from(rec, "radial", torch.float32), edges_from(rec, "angular", torch.float32)
    out = OM.forward(w, p, pos, types, [len(pos)], r, a)
    n = len(pos)
    for key, ours, tol in (("energies", out["energies"].numpy(), 1e-5),
                           ("forces", out["forces"].numpy(), 1e-4),
                           ("virial", out["virial"][0].numpy() / n, 1e-5)):
        scale = n if key == "virial" else 1
        f32, f64 = rec[f"{key}_f32"] / scale, rec[f"{key}_f64"] / scale
        bar = max(tol, 2.0 * np.abs(f32 - f64).max())
        assert np.abs(ours - f32).max() < bar, key


def test_message_block_matches_reference():
    p, w = load_weights("mp")
    rec = golden("block_mp_amo96")
    pos = torch.as_tensor(rec["positions"])
    r = edges_from(rec, "radial")
    vec = OM.edge_vectors(pos, r.center, r.neighbor, r.offsets)
    out = OM.message_block(w, "message_blocks.1.", p, torch.as_tensor(rec["hidden"]),
                           torch.as_tensor(rec["types"]), r.center, r.neighbor, vec)
    np.testing.assert_allclose(out.numpy(), rec["out_hidden"], rtol=1e-11, atol=1e-11)


def test_equivariant_block_and_encoder_match_reference():
    p, w = load_weights("eq")
    rec = golden("block_eq_amo96")
    pos = torch.as_tensor(rec["positions"])
    r = edges_from(rec, "radial")
    vec = OM.edge_vectors(pos, r.center, r.neighbor, r.offsets)
    lq = p["equivariant_l_max"]
    scale = OM.orthonormal_scale(lq, torch.float64)
    unit = vec / torch.linalg.vector_norm(vec, dim=-1, keepdim=True).clamp_min(1e-12)
    harm = OM.angular_basis(unit, lq, OM.z_tables(w, torch.float64)) * scale
    np.testing.assert_allclose(harm.numpy(), rec["harmonics"], rtol=1e-12, atol=1e-13)
    h, d = OM.equivariant_block(w, "message_blocks.1.", p, torch.as_tensor(rec["hidden"]),
                                torch.as_tensor(rec["direction"]), torch.as_tensor(rec["types"]),
                                r.center, r.neighbor, vec, harm)
    np.testing.assert_allclose(h.numpy(), rec["out_hidden"], rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(d.numpy(), rec["out_direction"], rtol=1e-11, atol=1e-11)
    mom = torch.as_tensor(rec["enc_moments"])
    enc = OM.direction_encoder(w, mom[..., :24] * scale, lq)
    np.testing.assert_allclose(enc.numpy(), rec["enc_out"], rtol=1e-12, atol=1e-13)


def test_nep_descriptor_matches_reference():
    rec = golden("nep_desc_pbte64")
    p = {"l_max": 4, "has_q_222": 1, "rcut_radial": 6.0, "rcut_angular": 4.0}
    w = {"descriptor.radial.c_table": torch.as_tensor(rec["c_radial"]),
         "descriptor.angular.c_table": torch.as_tensor(rec["c_angular"])}
    pos = torch.as_tensor(rec["positions"])
    _, _, _, q = OM._descriptor(w, p, pos, torch.as_tensor(rec["types"]),
                                edges_from(rec, "radial"), edges_from(rec, "angular"))
    np.testing.assert_allclose(q.numpy(), rec["q"], rtol=1e-11, atol=1e-12)
