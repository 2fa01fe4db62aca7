"""Test-only stand-in for ``ase.stress``."""

import numpy as np


def full_3x3_to_voigt_6_stress(stress):
    """Voigt order [xx, yy, zz, yz, xz, xy], off-diagonals symmetrised."""
    s = np.asarray(stress)
    return np.array([s[0, 0], s[1, 1], s[2, 2], (s[1, 2] + s[2, 1]) / 2,
                     (s[0, 2] + s[2, 0]) / 2, (s[0, 1] + s[1, 0]) / 2])
