"""Chemical element symbols and atomic numbers.

The reference resolves element symbols through ``ase.data``
(``rune/mobius/plugin.py:6``, ``rune/mobius/interface/batch.py:5``).  ASE is an
optional dependency here, so the periodic table is carried as plain data:
``CHEMICAL_SYMBOLS[Z]`` is the symbol of atomic number ``Z`` and index 0 holds
the placeholder ``"X"``, matching ASE's convention.
"""

from __future__ import annotations

CHEMICAL_SYMBOLS = (
    "X",
    "H", "He",
    "Li", "Be", "B", "C", "N", "O", "F", "Ne",
    "Na", "Mg", "Al", "Si", "P", "S", "Cl", "Ar",
    "K", "Ca", "Sc", "Ti", "V", "Cr", "Mn", "Fe", "Co", "Ni", "Cu", "Zn",
    "Ga", "Ge", "As", "Se", "Br", "Kr",
    "Rb", "Sr", "Y", "Zr", "Nb", "Mo", "Tc", "Ru", "Rh", "Pd", "Ag", "Cd",
    "In", "Sn", "Sb", "Te", "I", "Xe",
    "Cs", "Ba", "La", "Ce", "Pr", "Nd", "Pm", "Sm", "Eu", "Gd", "Tb", "Dy",
    "Ho", "Er", "Tm", "Yb", "Lu", "Hf", "Ta", "W", "Re", "Os", "Ir", "Pt",
    "Au", "Hg", "Tl", "Pb", "Bi", "Po", "At", "Rn",
    "Fr", "Ra", "Ac", "Th", "Pa", "U", "Np", "Pu", "Am", "Cm", "Bk", "Cf",
    "Es", "Fm", "Md", "No", "Lr", "Rf", "Db", "Sg", "Bh", "Hs", "Mt", "Ds",
    "Rg", "Cn", "Nh", "Fl", "Mc", "Lv", "Ts", "Og",
)

ATOMIC_NUMBERS = {symbol: number for number, symbol in enumerate(CHEMICAL_SYMBOLS)}


def symbol_of(number: int) -> str:
    """Symbol for ``number``; unknown numbers render as ``Z<n>`` like the reference."""
    if 0 <= number < len(CHEMICAL_SYMBOLS):
        return CHEMICAL_SYMBOLS[number]
    return f"Z{number}"
