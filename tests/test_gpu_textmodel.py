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
    """fp32 native outputs against the fp64 oracle on the same weights."""
    nl = ONB.build(s.positions, s.cell, s.pbc, params["rcut_radial"], params["rcut_angular"])
    sp = ONB.split(nl)
    mk = lambda k: OM.Edges(torch.as_tensor(sp[k][0]), torch.as_tensor(sp[k][1]),
                            torch.as_tensor(sp[k][2]))
    fwd = OM.nep_forward if nep else OM.forward
    ref = fwd(weights, params, torch.as_tensor(s.positions), torch.as_tensor(types).long(),
              [len(s)], mk("radial"), mk("angular"))
    de = (out["energies"].cpu().double() - ref["energies"]).abs().max().item()
    df = (out["forces"].cpu().double() - ref["forces"]).abs().max().item()
    dw = (out["virial"].cpu().double() - ref["virial"]).abs().max().item() / len(s)
    print(f"native vs fp64 oracle: dE {de:.1e} dF {df:.1e} dW/atom {dw:.1e}")
    assert de <= 1e-5 and df <= 1e-4 and dw <= 1e-5, (de, df, dw)


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
