"""ASE calculator and batch builder shared by the Möbius and NEP plugins.

``Calculator(artifact, device="cpu", compute_stress=True, **kwargs)``
mirrors ``rune/mobius/interface/calculator.py:14-98``: the same signature and
default, implemented properties, results (energy, free_energy, forces, Voigt
stress = -W/V) and errors (``PropertyNotImplementedError`` when stress is
disabled, ``ValueError`` for non-positive volume, unsupported elements and
neighbour overflow).  ``device`` is where the model module lives, as in the
reference; the neighbour search and the whole evaluation always run on a HIP
device (the given one when it is a ``cuda`` device, else the current one),
and there is no CPU evaluation path.

``BatchBuilder(params, device, dtype).build`` returns the reference's padded
batch dict (``rune/mobius/interface/batch.py:124-166``) on ``device``, built
from the GPU lists.  ASE is imported lazily; without ASE the array API in
``rune_amd.api`` works.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _native as N
from .elements import ATOMIC_NUMBERS, symbol_of


def _ase():
    try:
        from ase.calculators.calculator import Calculator as ASECalculator
        from ase.calculators.calculator import PropertyNotImplementedError, all_changes
    except ImportError as exc:  # pragma: no cover - depends on the environment
        raise ImportError("the ASE calculator needs the `ase` package; use rune_amd.api "
                          "for an ASE-free array interface") from exc
    return ASECalculator, PropertyNotImplementedError, all_changes


def voigt_from_3x3(stress):
    """``ase.stress.full_3x3_to_voigt_6_stress``: [xx, yy, zz, yz, xz, xy]."""
    s = np.asarray(stress)
    return np.array([s[0, 0], s[1, 1], s[2, 2], (s[1, 2] + s[2, 1]) / 2,
                     (s[0, 2] + s[2, 0]) / 2, (s[0, 1] + s[1, 0]) / 2])


class BatchBuilder:
    """Convert one structure to a reference-format batch (padded lists)."""

    def __init__(self, params, device, dtype, kind="Möbius"):
        self.device = torch.device(device) if device is not None else torch.device("cpu")
        self.compute_device = N.compute_device(self.device)
        self.dtype = dtype
        self.kind = kind
        self.elements = list(params["elements"])
        self.cutoff_radial = float(params["rcut_radial"])
        self.cutoff_angular = float(params["rcut_angular"])
        self.max_neighbors_radial = int(params["max_neighbors_radial"])
        self.max_neighbors_angular = int(params["max_neighbors_angular"])
        self.z_to_type = {ATOMIC_NUMBERS[e]: t for t, e in enumerate(self.elements)}
        self._cached = None
        self.nlist = N.NeighborList()

    def types_and_counts(self, numbers):
        """``_types_and_counts`` (batch.py:168-197) on the compute device; the
        last atomic-number tuple is cached."""
        numbers = tuple(int(z) for z in numbers)
        if self._cached is not None and self._cached[0] == numbers:
            return self._cached[1], self._cached[2]
        missing = sorted(set(numbers).difference(self.z_to_type))
        if missing:
            raise ValueError(
                f"Atoms contain elements not supported by this {self.kind} model: "
                f"{[symbol_of(z) for z in missing]}. "
                f"Model elements (type-id order): {self.elements}.")
        types = torch.tensor([self.z_to_type[z] for z in numbers], dtype=torch.long,
                             device=self.compute_device)
        counts = torch.tensor([len(numbers)], dtype=torch.long, device=self.compute_device)
        self._cached = (numbers, types, counts)
        return types, counts

    def neighbors(self, positions, cell, pbc):
        if self.cutoff_radial <= 0.0 or self.cutoff_angular <= 0.0:
            raise ValueError(f"{self.kind} radial and angular cutoffs must be positive.")
        pos = torch.as_tensor(np.asarray(positions, np.float64), device=self.compute_device)
        return self.nlist.build(pos, [0, len(positions)], [np.asarray(cell, np.float64)],
                                [np.broadcast_to(np.asarray(pbc, bool), (3,))],
                                self.cutoff_radial, self.cutoff_angular,
                                self.max_neighbors_radial, self.max_neighbors_angular)

    def build(self, atoms, *, compute_forces, compute_virial):
        types, counts = self.types_and_counts(atoms.numbers)
        n = len(atoms)
        nl = self.neighbors(atoms.positions, atoms.cell[:], atoms.pbc)
        rec = nl.export()
        dev = self.compute_device
        view = rec["view"].long()
        nbr = rec["nbr"].long()
        shift = rec["shift"].double()
        cell = torch.as_tensor(np.asarray(atoms.cell[:], np.float64), device=dev)
        # offsets S @ cell in fp64, the order of batch.py:76
        offsets = (shift[:, 0:1] * cell[0] + shift[:, 1:2] * cell[1]) + shift[:, 2:3] * cell[2]
        out = {"types": types.to(self.device), "n_atoms_per_structure": counts.to(self.device),
               "positions": torch.as_tensor(np.asarray(atoms.positions), dtype=self.dtype,
                                            device=self.device),
               "compute_forces": bool(compute_forces), "compute_virial": bool(compute_virial)}
        for kind, cols, cap in (("radial", (0, 1), self.max_neighbors_radial),
                                ("angular", (2, 3), self.max_neighbors_angular)):
            # each centre's records of this list fill the first slots of its
            # padded row, in record order (batch.py:9-39)
            begin, end = view[:, cols[0]], view[:, cols[1]]
            count = end - begin
            slot = torch.arange(cap, device=dev)
            live = slot[None, :] < count[:, None]
            src = (begin[:, None] + slot[None, :])[live]
            nb = torch.full((n, cap), -1, dtype=torch.long, device=dev)
            of = torch.zeros((n, cap, 3), dtype=torch.float64, device=dev)
            nb[live] = nbr[src]
            of[live] = offsets[src]
            out[f"{kind}_neighbors"] = nb.to(self.device)
            out[f"{kind}_offsets"] = of.to(device=self.device, dtype=self.dtype)
        return out


def make_calculator_class(load_model, family_name):
    ASECalculator, PropertyNotImplementedError, all_changes = _ase()

    class Calculator(ASECalculator):
        implemented_properties = ["energy", "free_energy", "forces", "stress"]

        def __init__(self, artifact, device="cpu", compute_stress=True, **kwargs):
            super().__init__(**kwargs)
            self.device = torch.device(device) if device is not None else torch.device("cpu")
            self.model = load_model(artifact, device=self.device)
            self.model.eval()
            self.model.requires_grad_(False)
            self.compute_stress = bool(compute_stress)
            self.implemented_properties = ["energy", "free_energy", "forces"]
            if self.compute_stress:
                self.implemented_properties.append("stress")
            dtype = next(self.model.parameters()).dtype
            self.batch_builder = BatchBuilder(self.model.params, self.device, dtype,
                                              family_name)

        def calculate(self, atoms=None, properties=None, system_changes=all_changes):
            properties = properties or ["energy"]
            super().calculate(atoms, properties, system_changes)
            atoms = atoms if atoms is not None else self.atoms
            if atoms is None:
                raise ValueError("Calculator requires an ASE Atoms object.")
            requested = set(properties)
            want_f = "forces" in requested
            want_w = "stress" in requested
            if want_w and not self.compute_stress:
                raise PropertyNotImplementedError(
                    "Stress is disabled for this Calculator. "
                    "Construct it with compute_stress=True for NPT or stress calculations.")
            volume = None
            if want_w:
                volume = atoms.get_volume()
                if volume <= 0:
                    raise ValueError("Stress calculation requires a positive cell volume.")
            types, _ = self.batch_builder.types_and_counts(atoms.numbers)
            nl = self.batch_builder.neighbors(atoms.positions, atoms.cell[:], atoms.pbc)
            out = self.model.native().compute(nl, types, 1, want_f, want_w)
            # fp32 kernel results, handed back in the model's dtype like the reference
            out = {k: v.to(self.batch_builder.dtype) for k, v in out.items()}
            energy = float(out["energy"][0].cpu())
            self.results = {"energy": energy, "free_energy": energy}
            if want_f:
                self.results["forces"] = out["forces"].cpu().numpy()
            if want_w:
                virial = out["virial"][0].cpu().numpy().reshape(3, 3)
                self.results["stress"] = voigt_from_3x3(-np.asarray(virial) / volume)

        def _build_batch(self, atoms, *, compute_forces=True, compute_virial=False):
            return self.batch_builder.build(atoms, compute_forces=compute_forces,
                                            compute_virial=compute_virial)

    return Calculator
