"""ASE-free array API of the HIP evaluator.

``Evaluator(params, state_dict, family)`` owns a native model handle and a
neighbour-list handle.  ``evaluate(structures)`` takes one or many
structures (objects with ``positions``, ``numbers``, ``cell``, ``pbc``) and
returns per-atom energies, per-structure energies, forces and virials as
device tensors -- the quantities of ``Mobius.forward`` / ``NEP.forward``
(``rune/mobius/model.py:307-393``) computed end to end on the GPU, including
the neighbour search.
"""

from __future__ import annotations

import weakref

import numpy as np
import torch

from . import _native as N
from . import ops
from .elements import ATOMIC_NUMBERS, symbol_of


class Prepared:
    """Device-resident inputs of one batch of structures."""

    def __init__(self, positions, types, struct_ptr, cells, pbc):
        self.positions = positions      # fp64 [N,3] device
        self.types = types              # int32 [N] device
        self.struct_ptr = struct_ptr    # int64 [B+1] host
        self.cells = cells              # fp64 [B,3,3] host
        self.pbc = pbc                  # int32 [B,3] host

    @property
    def n_atoms(self):
        return int(self.struct_ptr[-1])

    @property
    def n_structures(self):
        return len(self.struct_ptr) - 1


class Evaluator:
    def __init__(self, params, state_dict, family, device="cuda", model_name="model"):
        self.device = N.require_device(device)
        self.params = dict(params)
        self.family = family
        self.elements = list(params["elements"])
        self.model_name = model_name
        self.z_to_type = {ATOMIC_NUMBERS[e]: t for t, e in enumerate(self.elements)}
        self.native = N.NativeModel(params, state_dict, family)
        self.nlist = N.NeighborList()
        self._op_handle = None

    def types_of(self, numbers):
        numbers = [int(z) for z in numbers]
        missing = sorted(set(numbers).difference(self.z_to_type))
        if missing:
            kind = "Möbius" if self.family == N.FAMILY_MOBIUS else "NEP"
            raise ValueError(
                f"Atoms contain elements not supported by this {kind} model: "
                f"{[symbol_of(z) for z in missing]}. "
                f"Model elements (type-id order): {self.elements}.")
        return np.array([self.z_to_type[z] for z in numbers], dtype=np.int32)

    def prepare(self, structures):
        if not isinstance(structures, (list, tuple)):
            structures = [structures]
        pos = np.concatenate([np.asarray(s.positions, np.float64).reshape(-1, 3)
                              for s in structures]) if structures else np.zeros((0, 3))
        types = np.concatenate([self.types_of(s.numbers) for s in structures]) \
            if structures else np.zeros(0, np.int32)
        counts = [len(s.positions) for s in structures]
        sp = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
        cells = np.stack([np.asarray(s.cell, np.float64).reshape(3, 3) for s in structures])
        pbc = np.stack([np.broadcast_to(np.asarray(s.pbc, bool), (3,)).astype(np.int32)
                        for s in structures])
        return Prepared(torch.as_tensor(pos, device=self.device),
                        torch.as_tensor(types, device=self.device), sp, cells, pbc)

    def build_neighbors(self, prep):
        p = self.params
        self.nlist.build(prep.positions, prep.struct_ptr, prep.cells, prep.pbc,
                         p["rcut_radial"], p["rcut_angular"], p["max_neighbors_radial"],
                         p["max_neighbors_angular"])
        return self.nlist

    def evaluate(self, structures_or_prepared, compute_forces=True, compute_virial=True,
                 atom_virial=False):
        """E + F + virial through ``torch.ops.rune_hip.evaluate`` (see ``rune_amd.ops``)."""
        prep = structures_or_prepared
        if not isinstance(prep, Prepared):
            prep = self.prepare(prep)
        if atom_virial:
            nl = self.build_neighbors(prep)
            return self.native.compute(nl, prep.types, prep.n_structures, compute_forces,
                                       compute_virial, atom_virial)
        if self._op_handle is None:
            self._op_handle = ops.register(self)
            # finalize (not __del__) also runs at interpreter exit, before the
            # ops module is torn down
            weakref.finalize(self, ops.unregister, self._op_handle)
        e, etot, f, v = torch.ops.rune_hip.evaluate(
            self._op_handle, prep.positions, prep.types, [int(x) for x in prep.struct_ptr],
            [float(x) for x in np.asarray(prep.cells).reshape(-1)],
            [int(x) for x in np.asarray(prep.pbc).reshape(-1)], bool(compute_forces),
            bool(compute_virial))
        out = {"energies": e, "energy": etot}
        if compute_forces:
            out["forces"] = f
        if compute_virial:
            out["virial"] = v
        return out


def load_checkpoint(path):
    """``model.pt`` inference artifact -> (plugin name, params, state_dict).

    Loaded with ``weights_only=True``: only tensors and plain containers.
    """
    ck = torch.load(path, map_location="cpu", weights_only=True)
    return ck.get("plugin", {}).get("name"), ck["model_params"], ck["model_state_dict"]
