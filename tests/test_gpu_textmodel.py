"""Models read natively from text artifacts (``rune_model_load``) against the
same models built from their state dicts, and against the CPU oracle (needs
an MI355X; run with ``-m gpu``).

mobius1: the fixtures written by the reference's exporter
(``tests/golden/export_*.mobius.txt``, rune/mobius/export.py:120-146) against
this build's seeded models that produced them.  nep4 / nep4_zbl: files written
by the nep.txt writer, read natively and by the Python reader
(rune/nep/model.py:284-489 semantics).  Native and state-dict outputs must be
bitwise equal; the native outputs are also compared with the fp64 oracle
evaluating the weights as the text file holds them (fp32 tolerances).
"""

import numpy as np
import pytest
import torch

from oracle import model as OM
from oracle import neighbors as ONB
from rune_amd import workloads as W
from rune_amd.mobius import export as EX
from tests.golden.make_golden import small_export_model
from tests.helpers import GOLDEN

pytestmark = pytest.mark.gpu


def _outputs(model, s, types, rc_r, rc_a, max_r, max_a):
    from rune_amd import _native as N
    nl = N.NeighborList().build(torch.as_tensor(s.positions, device="cuda"), [0, len(s)],
                                [s.cell], [np.ones(3, np.int32)], rc_r, rc_a, max_r, max_a)
    return model.compute(nl, torch.as_tensor(types, device="cuda"), 1)


def _assert_equal(a, b):
    for k in ("energies", "energy", "forces", "virial"):
        assert torch.equal(a[k], b[k]), k


def _assert_matches_oracle(out, weights, params, s, types, nep=False):
    """fp32 native outputs against the oracle on the same weights: within the
    fp32 tolerances of the fp64 oracle, and of the oracle in fp32 (the
    reference's own fp32 path) widened by that path's distance from fp64."""
    nl = ONB.build(s.positions, s.cell, s.pbc, params["rcut_radial"], params["rcut_angular"])
    sp = ONB.split(nl)
    fwd = OM.nep_forward if nep else OM.forward

    def oracle(dtype):
        mk = lambda k: OM.Edges(torch.as_tensor(sp[k][0]), torch.as_tensor(sp[k][1]),
                                torch.as_tensor(sp[k][2], dtype=dtype))
        w = {k: v.to(dtype) if torch.is_tensor(v) and v.is_floating_point() else v
             for k, v in weights.items()}
        return fwd(w, params, torch.as_tensor(s.positions, dtype=dtype),
                   torch.as_tensor(types).long(), [len(s)], mk("radial"), mk("angular"))

    def dist(a, b):
        return ((a["energies"].double() - b["energies"].double()).abs().max().item(),
                (a["forces"].double() - b["forces"].double()).abs().max().item(),
                (a["virial"].double() - b["virial"].double()).abs().max().item() / len(s))

    r64, r32 = oracle(torch.float64), oracle(torch.float32)
    got = {k: out[k].cpu() for k in ("energies", "forces", "virial")}
    hip, ref, vs32 = dist(got, r64), dist(r32, r64), dist(got, r32)
    print(f"native - fp64 oracle {hip}; reference fp32 - fp64 {ref}; native - fp32 {vs32}")
    for h, r, v, t in zip(hip, ref, vs32, (1e-5, 1e-4, 1e-5)):
        assert h <= t, (hip, ref)
        assert v <= t + r, (vs32, ref)


@pytest.mark.parametrize("kind", ["local", "mp", "eq"])
def test_reference_exported_mobius_txt_loads_natively(kind):
    from rune_amd import _native as N
    model = small_export_model(kind)
    params = model.params
    native = N.NativeModel.load(GOLDEN / f"export_{kind}.mobius.txt")
    ref = N.NativeModel(params, model.state_dict(), N.FAMILY_MOBIUS)
    rc_r, rc_a, max_r, max_a = native.limits()
    assert (rc_r, rc_a) == (params["rcut_radial"], params["rcut_angular"])
    assert (max_r, max_a) == (params["max_neighbors_radial"], params["max_neighbors_angular"])
    assert [native.element(t) for t in range(2)] == ["Fe", "C"]
    s = W.si_diamond(seed=41, reps=2, a=4.2)
    types = np.arange(len(s)) % 2
    out = _outputs(native, s, types, rc_r, rc_a, max_r, max_a)
    _assert_equal(out, _outputs(ref, s, types, rc_r, rc_a, max_r, max_a))
    # the weights exactly as the file holds them (float64 text of float32 values)
    _, _, _, tensors = EX.read_mobius_txt(GOLDEN / f"export_{kind}.mobius.txt")
    weights = {k: v for k, v in tensors.items() if not k.startswith("desc.")}
    _assert_matches_oracle(out, weights, params, s, types)


def _nep_variant(tmp_path, variant):
    from rune_amd.nep.model import seeded_nep
    path = tmp_path / "nep.txt"
    seeded_nep(seed=7).save_nep_txt(path)
    text = path.read_text()
    head, rest = text.split("\n", 1)
    if variant == "universal_zbl":
        text = head.replace("nep4", "nep4_zbl") + "\nzbl 1.5 2.5\n" + rest
    elif variant == "flexible_zbl":
        rows = [[1.4 + 0.1 * k, 2.5, 0.18175, 3.1998, 0.50986, 0.94229, 0.28022, 0.4029,
                 0.02817, 0.20162] for k in range(3)]
        text = (head.replace("nep4", "nep4_zbl") + "\nzbl 0 0\n" + rest +
                "".join(f"{v:18.10e}\n" for r in rows for v in r))
    path.write_text(text)
    return path


@pytest.mark.parametrize("variant", ["plain", "universal_zbl", "flexible_zbl"])
def test_nep_txt_loads_natively(variant, tmp_path):
    from rune_amd import _native as N
    from rune_amd.nep.model import NEP
    path = _nep_variant(tmp_path, variant)
    model = NEP.from_nep_txt(path)
    native = N.NativeModel.load(path)
    ref = N.NativeModel(model.params, model.state_dict(), N.FAMILY_NEP)
    rc_r, rc_a, max_r, max_a = native.limits()
    assert (max_r, max_a) == (100, 30)
    s = W.rocksalt(seed=42, reps=2, a=4.6)   # nearest neighbours 2.3 A: inside the ZBL taper
    types = np.array([0 if z == 82 else 1 for z in s.numbers], np.int32)
    out = _outputs(native, s, types, rc_r, rc_a, max_r, max_a)
    _assert_equal(out, _outputs(ref, s, types, rc_r, rc_a, max_r, max_a))
    weights = {k: v.detach().double() if v.is_floating_point() else v
               for k, v in model.state_dict().items()}
    _assert_matches_oracle(out, weights, model.params, s, types, nep=True)
