"""Test-only stand-in for ``ase.calculators.calculator``.

``Calculator.get_property`` follows ASE's contract as the reference
calculator relies on it: a property outside ``implemented_properties`` raises
``PropertyNotImplementedError`` before any calculation; otherwise the
calculation runs when the atoms changed since the last one (positions,
numbers, cell, pbc) or the property is not among the cached results.
``calculate`` stores a copy of the atoms it was called with.
"""

import numpy as np

all_changes = ["positions", "numbers", "cell", "pbc", "initial_charges", "initial_magmoms"]


class PropertyNotImplementedError(NotImplementedError):
    pass


class Calculator:
    implemented_properties: list = []

    def __init__(self, **kwargs):
        self.parameters = dict(kwargs)
        self.atoms = None
        self.results = {}

    def _changes(self, atoms):
        if self.atoms is None:
            return list(all_changes)
        out = []
        if not np.array_equal(self.atoms.positions, atoms.positions):
            out.append("positions")
        if not np.array_equal(self.atoms.numbers, atoms.numbers):
            out.append("numbers")
        if not np.array_equal(self.atoms.cell.array, atoms.cell.array):
            out.append("cell")
        if not np.array_equal(self.atoms.pbc, atoms.pbc):
            out.append("pbc")
        return out

    def calculate(self, atoms=None, properties=("energy",), system_changes=all_changes):
        if atoms is not None:
            self.atoms = atoms.copy()

    def get_property(self, name, atoms=None):
        if name not in self.implemented_properties:
            raise PropertyNotImplementedError(f"{name} property not implemented")
        atoms = atoms if atoms is not None else self.atoms
        changes = self._changes(atoms)
        if changes:
            self.results = {}
        if name not in self.results:
            self.calculate(atoms, [name], changes)
        return self.results[name]
