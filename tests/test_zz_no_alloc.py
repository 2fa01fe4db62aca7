"""``rune_model_compute_static``: the evaluation with its workspace in the
library's static device scratch (no device allocation), against
``rune_model_compute`` through the C ABI.  Same kernels, same order: outputs
must be bitwise equal, on two calls in a row with the second input smaller
(the scratch keeps the first call's contents), for every model family.  An
input whose workspace exceeds the scratch is refused with an error and
leaves the outputs untouched.  Needs an MI355X; run with ``-m gpu``."""

import numpy as np
import pytest
import torch

from rune_amd import workloads as W
from tests.helpers import load_weights

pytestmark = pytest.mark.gpu

KEYS = ("energies", "energy", "forces", "virial", "atom_virial")


def _cases(name):
    if name == "loc":
        return [W.si_diamond(seed=71, reps=3), W.si_diamond(seed=72, reps=1)]
    if name == "mp":
        return [W.fcc_alloy(seed=73, reps=2), W.amorphous(seed=74, n_atoms=14)]
    if name == "eq":
        return [W.amorphous(seed=75, n_atoms=60), W.amorphous(seed=76, n_atoms=24)]
    return [W.rocksalt(seed=77, reps=2), W.rocksalt(seed=78, reps=1)]


def _evaluator(name):
    from rune_amd import _native as N
    from rune_amd.api import Evaluator
    if name == "nep":
        from rune_amd.nep.model import seeded_nep
        model = seeded_nep(seed=5)
        return Evaluator(model.params, model.state_dict(), N.FAMILY_NEP)
    p, w = load_weights(name, torch.float32)
    return Evaluator(p, w, N.FAMILY_MOBIUS)


@pytest.mark.parametrize("name", ["loc", "mp", "eq", "nep"])
def test_static_entry_matches_allocating_entry(name):
    ev = _evaluator(name)
    for s in _cases(name):
        prep = ev.prepare(s)
        nl = ev.build_neighbors(prep)
        ref = ev.native.compute(nl, prep.types, 1, True, True, atom_virial=True)
        got = ev.native.compute(nl, prep.types, 1, True, True, atom_virial=True, static=True)
        torch.cuda.synchronize()
        print(f"{name}: {len(s)} atoms, {nl.n_records} records, "
              f"allocating workspace {ev.native.workspace_bytes()} bytes")
        for k in KEYS:
            assert torch.equal(got[k], ref[k]), (name, len(s), k)


def test_static_entry_refuses_a_workspace_beyond_the_scratch():
    from rune_amd import _native as N
    ev = _evaluator("eq")
    s = W.amorphous(seed=79, n_atoms=2000)
    prep = ev.prepare(s)
    nl = ev.build_neighbors(prep)
    limit = int(N.library().rune_model_static_scratch_bytes())
    assert limit == 64 << 20
    with pytest.raises(ValueError, match="static scratch holds 67108864"):
        ev.native.compute(nl, prep.types, 1, True, True, static=True)
    # the allocating entry point still evaluates it, and a small input after
    # the refusal goes through the static one again
    ev.native.compute(nl, prep.types, 1, True, True)
    small = ev.prepare(W.amorphous(seed=80, n_atoms=20))
    nl2 = ev.build_neighbors(small)
    a = ev.native.compute(nl2, small.types, 1, True, True, static=True)
    b = ev.native.compute(nl2, small.types, 1, True, True)
    for k in ("energies", "forces", "virial"):
        assert torch.equal(a[k], b[k]), k
