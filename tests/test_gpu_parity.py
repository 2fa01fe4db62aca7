"""HIP path vs the CPU oracle (needs an MI355X; run with ``-m gpu``)."""

import numpy as np
import pytest
import torch

from oracle import model as OM
from oracle import neighbors as ONB
from rune_amd import workloads as W
from tests.helpers import load_weights

pytestmark = pytest.mark.gpu

SMALL = {
    "si8": lambda: W.si_diamond(seed=21, reps=1),
    "si64": lambda: W.si_diamond(seed=22, reps=2),
    "fcc108": lambda: W.fcc_alloy(seed=23, reps=3),
    "pbte64": lambda: W.rocksalt(seed=24, reps=2),
}


def _fec4():
    cell = np.array([[4.1, .1, .2], [.0, 4.3, .1], [.1, .0, 4.5]])
    frac = np.array([[.10, .13, .22], [.82, .21, .37], [.30, .75, .19], [.68, .63, .81]])
    return W.Structure(frac @ cell, np.array([26, 6, 26, 6]), cell)


def _structures():
    out = {k: f() for k, f in SMALL.items()}
    out["fec4"] = _fec4()
    out["amo200"] = W.amorphous(seed=25, n_atoms=200)
    return out


def _evaluator(name, dtype=torch.float32):
    from rune_amd.api import Evaluator
    from rune_amd import _native as N
    p, w = load_weights(name, torch.float32)
    return Evaluator(p, w, N.FAMILY_MOBIUS), p


@pytest.mark.parametrize("name", ["si8", "si64", "fcc108", "pbte64", "fec4", "amo200"])
@pytest.mark.parametrize("rc", [(6.0, 5.0), (3.8, 3.5), (4.0, 6.5)])
def test_neighbor_list_bit_exact(name, rc):
    from rune_amd import _native as N
    s = _structures()[name]
    ref = ONB.build(s.positions, s.cell, s.pbc, rc[0], rc[1])
    nl = N.NeighborList().build(torch.as_tensor(s.positions, device="cuda"), [0, len(s)],
                                [s.cell], [s.pbc], rc[0], rc[1], 100000, 100000)
    out = {k: v.cpu().numpy() for k, v in nl.export().items()}
    assert nl.n_records == len(ref["neighbor"])
    np.testing.assert_array_equal(out["ptr"], ref["ptr"])
    np.testing.assert_array_equal(out["nbr"], ref["neighbor"])
    np.testing.assert_array_equal(out["shift"], ref["shift"])
    np.testing.assert_array_equal(out["vec"][:, :3], ref["vec32"])
    counts_r = np.bincount(ref["center"][ref["radial_mask"]], minlength=len(s))
    counts_a = np.bincount(ref["center"][ref["angular_mask"]], minlength=len(s))
    np.testing.assert_array_equal(out["view"][:, 1] - out["view"][:, 0], counts_r)
    np.testing.assert_array_equal(out["view"][:, 3] - out["view"][:, 2], counts_a)


def test_neighbor_list_dense_rows_after_sparse_build():
    """One list handle rebuilt from a sparse system (8 records per centre) to
    dense ones (160-183 records per centre, cutoffs beyond half the cell, so
    several images of an atom): every list bit for bit the oracle's."""
    from rune_amd import _native as N
    nl = N.NeighborList()
    cases = [(SMALL["si8"](), (3.8, 3.5)),
             (W.amorphous(seed=25, n_atoms=200), (8.0, 7.0)),
             (W.amorphous(seed=26, n_atoms=200), (8.0, 7.0))]
    for s, rc in cases:
        ref = ONB.build(s.positions, s.cell, s.pbc, rc[0], rc[1])
        nl.build(torch.as_tensor(s.positions, device="cuda"), [0, len(s)], [s.cell], [s.pbc],
                 rc[0], rc[1], 100000, 100000)
        out = {k: v.cpu().numpy() for k, v in nl.export().items()}
        print("rows", np.diff(ref["ptr"]).max(), "records", len(ref["neighbor"]), flush=True)
        assert nl.n_records == len(ref["neighbor"])
        np.testing.assert_array_equal(out["ptr"], ref["ptr"])
        np.testing.assert_array_equal(out["nbr"], ref["neighbor"])
        np.testing.assert_array_equal(out["shift"], ref["shift"])
        np.testing.assert_array_equal(out["vec"][:, :3], ref["vec32"])


def _oracle(p, w, s, types, dtype):
    nl = ONB.build(s.positions, s.cell, s.pbc, p["rcut_radial"], p["rcut_angular"])
    sp = ONB.split(nl)
    mk = lambda k: OM.Edges(torch.as_tensor(sp[k][0]), torch.as_tensor(sp[k][1]),
                            torch.as_tensor(sp[k][2], dtype=dtype))
    wd = {k: (v.to(dtype) if v.is_floating_point() else v) for k, v in w.items()}
    return OM.forward(wd, p, torch.as_tensor(s.positions, dtype=dtype),
                      torch.as_tensor(types, dtype=torch.long), [len(s)], mk("radial"),
                      mk("angular"))


def _compare(out, ref, n):
    e = out["energies"].cpu().double().numpy()
    f = out["forces"].cpu().double().numpy()
    v = out["virial"].cpu().double().numpy()[0]
    de = np.abs(e - ref["energies"].double().numpy()).max()
    df = np.abs(f - ref["forces"].double().numpy()).max()
    dv = np.abs(v - ref["virial"][0].double().numpy()).max() / n
    return de, df, dv


TOL = (1e-5, 1e-4, 1e-5)   # eV per atom, eV/Å max-abs, eV/atom (virial)


def assert_within(out, r64, r32, n, label="", tol=TOL):
    """The stated fp32 tolerances, asserted two ways for E, F and W/atom.

    * against the fp64 oracle: |HIP - fp64| <= max(tol, 2 |ref32 - fp64|);
    * against the reference's own fp32 path (the oracle in fp32, op for op):
      |HIP - ref32| <= tol + |ref32 - fp64|.
    The widening by |ref32 - fp64| matters only where that path is itself
    further than the tolerance from exact arithmetic (heavy-element cells
    with large descriptors).  All three distances are printed.
    """
    gpu = _compare(out, r64, n)
    ref = _compare(r32, r64, n)
    vs32 = _compare(out, r32, n)
    print(f"{label} HIP-fp64 {['%.2e' % x for x in gpu]}  ref32-fp64 "
          f"{['%.2e' % x for x in ref]}  HIP-ref32 {['%.2e' % x for x in vs32]}", flush=True)
    for g, r, v, t in zip(gpu, ref, vs32, tol):
        assert g <= max(t, 2.0 * r), (label, gpu, ref)
        assert v <= t + r, (label, vs32, ref)
    return gpu, ref


def check_against_oracle(model, out, s, types):
    """fp32 HIP result vs the oracle in fp64 and fp32 (`assert_within`)."""
    p, w64 = load_weights(model, torch.float64)
    _, w32 = load_weights(model, torch.float32)
    r64 = _oracle(p, w64, s, types, torch.float64)
    r32 = _oracle(p, w32, s, types, torch.float32)
    gpu, ref = assert_within(out, r64, r32, len(s), model)
    de_tot = abs(float(out["energy"][0]) - float(r64["energy"][0]))
    assert de_tot <= max(1e-5 * len(s), 2.0 * abs(float(r32["energy"][0]) - float(r64["energy"][0])))
    return gpu, ref


@pytest.mark.parametrize("name", ["si8", "si64", "fcc108", "fec4", "amo200"])
def test_local_model_matches_oracle(name):
    ev, p = _evaluator("loc")
    s = _structures()[name]
    out = ev.evaluate(s)
    check_against_oracle("loc", out, s, ev.types_of(s.numbers))


def test_local_model_is_deterministic():
    ev, _ = _evaluator("loc")
    s = _structures()["amo200"]
    a = ev.evaluate(s)
    b = ev.evaluate(s)
    for k in ("energies", "energy", "forces", "virial"):
        assert torch.equal(a[k], b[k]), k


def _nep_oracle(model, s, dtype):
    p = model.params
    w = {k: (v.detach().to(dtype) if v.is_floating_point() else v) for k, v in
         model.state_dict().items()}
    types = (s.numbers == 52).astype(np.int64) if "Te" in p["elements"] else None
    nl = ONB.build(s.positions, s.cell, s.pbc, p["rcut_radial"], p["rcut_angular"])
    sp = ONB.split(nl)
    mk = lambda k: OM.Edges(torch.as_tensor(sp[k][0]), torch.as_tensor(sp[k][1]),
                            torch.as_tensor(sp[k][2], dtype=dtype))
    return OM.nep_forward(w, p, torch.as_tensor(s.positions, dtype=dtype),
                          torch.as_tensor(types), [len(s)], mk("radial"), mk("angular"))


@pytest.mark.parametrize("reps", [2, 3])
def test_nep_matches_oracle(reps):
    from rune_amd import _native as N
    from rune_amd.api import Evaluator
    from rune_amd.nep.model import seeded_nep
    model = seeded_nep(seed=0)
    ev = Evaluator(model.params, model.state_dict(), N.FAMILY_NEP)
    s = W.rocksalt(seed=30 + reps, reps=reps)
    out = ev.evaluate(s)
    r64 = _nep_oracle(model, s, torch.float64)
    r32 = _nep_oracle(model, s, torch.float32)
    assert_within(out, r64, r32, len(s), f"NEP {len(s)}")


def test_drop_in_model_forward_on_padded_batch():
    """``Mobius.forward(batch)`` with the reference's padded batch format."""
    from rune_amd.mobius.plugin import load_model
    from rune_amd import MODELS
    model = load_model(MODELS["mobius-oam-loc"], device="cuda").eval()
    s = W.si_diamond(seed=31, reps=2)
    p = model.params
    nl = ONB.build(s.positions, s.cell, s.pbc, p["rcut_radial"], p["rcut_angular"])
    sp = ONB.split(nl)
    rn, ro = ONB.pack(*sp["radial"], len(s), 64)
    an, ao = ONB.pack(*sp["angular"], len(s), 64)
    dev = torch.device("cuda")
    batch = {"positions": torch.as_tensor(s.positions, dtype=torch.float32, device=dev),
             "types": torch.full((len(s),), 13, dtype=torch.long, device=dev),
             "radial_neighbors": torch.as_tensor(rn, device=dev),
             "radial_offsets": torch.as_tensor(ro, dtype=torch.float32, device=dev),
             "angular_neighbors": torch.as_tensor(an, device=dev),
             "angular_offsets": torch.as_tensor(ao, dtype=torch.float32, device=dev),
             "n_atoms_per_structure": torch.tensor([len(s)], device=dev)}
    out = model(batch)
    check_against_oracle("loc", out, s, np.full(len(s), 13))
    f_only = model({**batch, "compute_virial": False})
    assert "virial" not in f_only and "forces" in f_only
    e_only = model({**batch, "compute_forces": False, "compute_virial": False})
    torch.testing.assert_close(e_only["energies"], out["energies"], rtol=0, atol=0)


def test_batched_structures_match_single_calls():
    ev, p = _evaluator("loc")
    cells = [W.si_diamond(seed=40 + k, reps=1 + (k % 2)) for k in range(4)]
    batched = ev.evaluate(cells)
    off = 0
    for k, s in enumerate(cells):
        single = ev.evaluate(s)
        n = len(s)
        torch.testing.assert_close(batched["energies"][off:off + n], single["energies"],
                                   rtol=0, atol=2e-6)
        torch.testing.assert_close(batched["forces"][off:off + n], single["forces"],
                                   rtol=0, atol=2e-5)
        torch.testing.assert_close(batched["virial"][k], single["virial"][0], rtol=1e-5,
                                   atol=1e-4)
        off += n


def test_errors_are_reported():
    from rune_amd import _native as N
    ev, p = _evaluator("loc")
    s = W.si_diamond(seed=1, reps=2)
    with pytest.raises(ValueError, match="not supported"):
        ev.types_of([13, 2000])
    nl = N.NeighborList()
    with pytest.raises(ValueError, match="exceeds max_neighbors=10"):
        nl.build(torch.as_tensor(s.positions, device="cuda"), [0, len(s)], [s.cell], [s.pbc],
                 6.0, 5.0, 10, 100)


@pytest.mark.parametrize("model,reps", [("loc", 2), ("loc", 11), ("mp", 3)])
def test_out_of_range_type_is_reported_and_cleared(model, reps):
    """A type outside [0, n_types) is reported by the device check (the kernels
    read a clamped copy meanwhile), and the next call with valid types is
    unaffected: bitwise equal to the call before.  64 atoms: one checking
    block; 10,648: a grid; the MP model also runs work on its side stream,
    which the failed call still joins."""
    from rune_amd import _native as N
    ev, p = _evaluator(model)
    s = W.si_diamond(seed=3, reps=reps)
    types = torch.as_tensor(ev.types_of(s.numbers), device="cuda")
    nl = N.NeighborList().build(torch.as_tensor(s.positions, device="cuda"), [0, len(s)],
                                [s.cell], [np.ones(3, np.int32)], p["rcut_radial"],
                                p["rcut_angular"], p["max_neighbors_radial"],
                                p["max_neighbors_angular"])
    good = ev.native.compute(nl, types, 1, True, True)
    for bad in (-1, 1 << 20):
        t = types.clone()
        t[len(s) // 2] = bad
        with pytest.raises(ValueError, match="outside"):
            ev.native.compute(nl, t, 1, True, True)
    again = ev.native.compute(nl, types, 1, True, True)
    for k in ("energies", "energy", "forces", "virial"):
        assert torch.equal(good[k], again[k]), k


@pytest.mark.parametrize("name", ["fec4", "fcc108", "amo200"])
def test_mp_model_matches_oracle(name):
    ev, p = _evaluator("mp")
    s = _structures()[name]
    out = ev.evaluate(s)
    check_against_oracle("mp", out, s, ev.types_of(s.numbers))


def _small_model(seed, **changes):
    from rune_amd.mobius.model import Mobius
    from rune_amd.mobius.plugin import resolve_params
    values = {"elements": ["Fe", "C", "O"], "hidden_dim": 16, "blocks": 1, "ffn_dim": 24,
              "message_layers": 2, "message_dim": 12, "message_groups": 4, "pair_dim": 3,
              "vector_channels": 3, "message_basis_size": 5, "rcut_radial": 4.8,
              "rcut_angular": 4.4, "n_max_radial": 2, "n_max_angular": 2,
              "basis_size_radial": 3, "basis_size_angular": 3, "l_max": 4, "l_max_4body": 2,
              "l_max_5body": 1, "has_q_112": 1, "has_q_123": 1, "has_q_233": 1, "has_q_134": 1,
              "max_neighbors_radial": 200, "max_neighbors_angular": 200}
    values.update(changes)
    torch.manual_seed(seed)
    model = Mobius(resolve_params(values))
    with torch.no_grad():     # non-trivial norm weights and scaler
        for name, t in model.named_parameters():
            if name.endswith("norm.weight"):
                t.uniform_(0.5, 1.5)
        model.q_scaler.uniform_(0.5, 1.5)
    return model


@pytest.mark.parametrize("changes", [
    {}, {"vector_channels": 0}, {"activation": "tanh"}, {"activation": "gelu"},
    {"message_cutoff": 3.9, "message_basis_size": 4},
    {"rcut_angular": 5.2, "zbl": [0.8, 1.6]},
    # widths of the fused edge-MLP kernels and the contiguous-column record
    # kernels: D 32 / 64 / 128, one or two gate blocks, basis 4 / 17 / 20
    # (drb tail rows 4 / 1 / 4), hidden 64 / 128 / 256
    {"hidden_dim": 64, "message_dim": 32, "message_groups": 4, "vector_channels": 4,
     "message_basis_size": 4},
    {"hidden_dim": 128, "message_dim": 64, "message_groups": 8, "vector_channels": 20,
     "message_basis_size": 20, "activation": "tanh"},
    {"hidden_dim": 256, "message_dim": 128, "message_groups": 16, "vector_channels": 8,
     "message_basis_size": 17, "activation": "gelu"},
    # fallbacks: basis 5 (drb tail of 5 rows), 34 gates, groups narrower than a lane's columns
    {"hidden_dim": 64, "message_dim": 32, "message_groups": 4, "vector_channels": 4,
     "message_basis_size": 5},
    {"hidden_dim": 64, "message_dim": 96, "message_groups": 32, "vector_channels": 2},
])
def test_small_mp_variants_match_oracle(changes):
    from rune_amd import _native as N
    from rune_amd.api import Evaluator
    model = _small_model(5, **changes)
    p = model.params
    rng = np.random.default_rng(3)
    cell = np.diag([6.1, 6.4, 6.7]) + rng.uniform(-0.4, 0.4, (3, 3))
    s = W.Structure(rng.random((14, 3)) @ cell, rng.choice([26, 6, 8], 14), cell)
    ev = Evaluator(p, model.state_dict(), N.FAMILY_MOBIUS)
    out = ev.evaluate(s)
    types = ev.types_of(s.numbers)
    sd = model.state_dict()
    w64 = {k: v.double() if v.is_floating_point() else v for k, v in sd.items()}
    r64 = _oracle(p, w64, s, types, torch.float64)
    w32 = {k: v.float() if v.is_floating_point() else v for k, v in sd.items()}
    r32 = _oracle(p, w32, s, types, torch.float32)
    assert_within(out, r64, r32, len(s), str(changes))


@pytest.mark.parametrize("name", ["fec4", "fcc108", "amo200"])
def test_eq_model_matches_oracle(name):
    ev, p = _evaluator("eq")
    s = _structures()[name]
    out = ev.evaluate(s)
    check_against_oracle("eq", out, s, ev.types_of(s.numbers))


@pytest.mark.parametrize("name", ["fcc108", "amo200"])
def test_eq_model_with_tall_product_tiles_matches_oracle(name, monkeypatch):
    """The 64x96 tile the per-record GEMMs of cells with millions of records
    take (gate product N = 264, its transpose N = 192), run here on small
    cells by lowering the row threshold."""
    monkeypatch.setenv("RUNE_TALL_ROWS", "1")
    ev, p = _evaluator("eq")
    s = _structures()[name]
    out = ev.evaluate(s)
    check_against_oracle("eq", out, s, ev.types_of(s.numbers))


def _check_small(model):
    from rune_amd import _native as N
    from rune_amd.api import Evaluator
    p = model.params
    rng = np.random.default_rng(4)
    cell = np.diag([6.1, 6.4, 6.7]) + rng.uniform(-0.4, 0.4, (3, 3))
    s = W.Structure(rng.random((14, 3)) @ cell, rng.choice([26, 6, 8], 14), cell)
    ev = Evaluator(p, model.state_dict(), N.FAMILY_MOBIUS)
    out = ev.evaluate(s)
    types = ev.types_of(s.numbers)
    sd = model.state_dict()
    w64 = {k: v.double() if v.is_floating_point() else v for k, v in sd.items()}
    w32 = {k: v.float() if v.is_floating_point() else v for k, v in sd.items()}
    r64 = _oracle(p, w64, s, types, torch.float64)
    r32 = _oracle(p, w32, s, types, torch.float32)
    assert_within(out, r64, r32, len(s))


@pytest.mark.parametrize("changes", [
    {}, {"equivariant_l_max": 1}, {"equivariant_l_max": 2}, {"activation": "gelu"},
    {"message_cutoff": 3.9}, {"rcut_angular": 5.2, "zbl": [0.8, 1.6]},
    {"equivariant_channels": 5, "message_groups": 2},
])
def test_small_eq_variants_match_oracle(changes):
    base = {"message_mode": "equivariant", "equivariant_channels": 3}
    base.update(changes)
    _check_small(_small_model(6, **base))
