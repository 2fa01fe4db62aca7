"""Test-only stand-in for ``ase.Atoms`` (see ../README.txt).

Covers what the calculator tests use: chemical formulas such as "FeCFeC" or
"H2", Cartesian or scaled positions, a cell given as lengths or a 3x3
matrix, ``pbc`` (default False, as in ASE), ``get_volume``, per-atom access
with a settable ``symbol``, ``copy`` and the ``calc`` property getters.
"""

from __future__ import annotations

import re

import numpy as np

from .data import atomic_numbers, chemical_symbols

__all__ = ["Atoms", "Atom"]


def _parse_formula(formula):
    numbers = []
    for symbol, count in re.findall(r"([A-Z][a-z]?)(\d*)", formula):
        numbers += [atomic_numbers[symbol]] * (int(count) if count else 1)
    return numbers


class _Cell:
    def __init__(self, array):
        self.array = np.array(array, dtype=np.float64).reshape(3, 3)

    def __getitem__(self, item):
        return self.array[item]

    def __array__(self, dtype=None, copy=None):
        return self.array if dtype is None else self.array.astype(dtype)

    def volume(self):
        return float(abs(np.linalg.det(self.array)))


class Atom:
    def __init__(self, atoms, index):
        self._atoms, self._index = atoms, index

    @property
    def symbol(self):
        return chemical_symbols[int(self._atoms.numbers[self._index])]

    @symbol.setter
    def symbol(self, value):
        self._atoms.numbers[self._index] = atomic_numbers[value]


class Atoms:
    def __init__(self, symbols=None, positions=None, numbers=None, cell=None, pbc=False,
                 scaled_positions=None, calculator=None):
        if numbers is None:
            numbers = _parse_formula(symbols) if isinstance(symbols, str) else \
                [atomic_numbers[s] for s in (symbols or [])]
        self.numbers = np.array(numbers, dtype=np.int64)
        c = np.zeros((3, 3)) if cell is None else np.asarray(cell, dtype=np.float64)
        self.cell = _Cell(np.diag(c) if c.shape == (3,) else c)
        self.pbc = np.broadcast_to(np.asarray(pbc, dtype=bool), (3,)).copy()
        if scaled_positions is not None:
            positions = np.asarray(scaled_positions, dtype=np.float64) @ self.cell.array
        if positions is None:
            positions = np.zeros((len(self.numbers), 3))
        self.positions = np.array(positions, dtype=np.float64).reshape(-1, 3)
        self.calc = calculator

    def __len__(self):
        return len(self.numbers)

    def __getitem__(self, index):
        return Atom(self, index)

    def set_cell(self, cell, scale_atoms=False):
        c = np.asarray(cell, dtype=np.float64)
        new = np.diag(c) if c.shape == (3,) else c
        if scale_atoms:
            self.positions = self.positions @ np.linalg.solve(self.cell.array, new)
        self.cell = _Cell(new)

    def get_volume(self):
        return self.cell.volume()

    def copy(self):
        other = Atoms(numbers=self.numbers.copy(), positions=self.positions.copy(),
                      cell=self.cell.array.copy(), pbc=self.pbc.copy())
        return other

    def _get(self, name):
        if self.calc is None:
            raise RuntimeError("Atoms object has no calculator.")
        return self.calc.get_property(name, self)

    def get_potential_energy(self):
        return self._get("energy")

    def get_forces(self):
        return np.array(self._get("forces"))

    def get_stress(self):
        return np.array(self._get("stress"))
