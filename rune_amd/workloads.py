"""Seeded synthetic structures for the benchmark and parity configurations.

Every generator uses ``numpy.random.Generator(PCG64(seed))`` and returns
plain arrays (no ASE): a :class:`Structure` or a list of them.

* ``si_diamond``      C1: Si diamond cubic a = 5.43 Å, 4x4x4, sigma = 0.05 Å.
* ``rocksalt``        C2: rock salt (default PbTe) a = 6.46 Å, 12^3, sigma = 0.05 Å.
* ``fcc_alloy``       C3: 5-element equiatomic FCC a = 3.6 Å, 17^3, sigma = 0.1 Å.
* ``amorphous``       C4: cubic periodic cell at 0.08 atoms/Å^3, random sequential
                      placement with minimum image separation 1.8 Å, 10 elements.
* ``small_cells``     C5: 256 random triclinic cells of 8..64 atoms.
"""

from __future__ import annotations

import hashlib
import math
from dataclasses import dataclass, field

import numpy as np

from .elements import ATOMIC_NUMBERS

# The 89 elements of the OAM checkpoints, in type order.
OAM_ELEMENTS = (
    "H He Li Be B C N O F Ne Na Mg Al Si P S Cl Ar K Ca Sc Ti V Cr Mn Fe Co Ni Cu Zn "
    "Ga Ge As Se Br Kr Rb Sr Y Zr Nb Mo Tc Ru Rh Pd Ag Cd In Sn Sb Te I Xe Cs Ba La Ce "
    "Pr Nd Pm Sm Eu Gd Tb Dy Ho Er Tm Yb Lu Hf Ta W Re Os Ir Pt Au Hg Tl Pb Bi Ac Th "
    "Pa U Np Pu"
).split()


@dataclass
class Structure:
    positions: np.ndarray          # [N, 3] float64, Å
    numbers: np.ndarray            # [N] int64 atomic numbers
    cell: np.ndarray               # [3, 3] float64, rows are lattice vectors
    pbc: tuple = (True, True, True)
    info: dict = field(default_factory=dict)

    def __len__(self):
        return len(self.positions)

    @property
    def volume(self):
        return float(abs(np.linalg.det(self.cell)))

    def digest(self):
        h = hashlib.sha256()
        for a in (self.positions, self.numbers, self.cell):
            h.update(np.ascontiguousarray(a).tobytes())
        return h.hexdigest()


def _rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def _lattice(basis, reps, a):
    reps = np.asarray(reps)
    grid = np.stack(np.meshgrid(*[np.arange(r) for r in reps], indexing="ij"), -1).reshape(-1, 3)
    frac = (grid[:, None, :] + np.asarray(basis)[None, :, :]).reshape(-1, 3)
    return frac * a


FCC = [(0, 0, 0), (0, 0.5, 0.5), (0.5, 0, 0.5), (0.5, 0.5, 0)]


def si_diamond(seed=1, reps=4, a=5.43, sigma=0.05):
    basis = FCC + [(x + 0.25, y + 0.25, z + 0.25) for x, y, z in FCC]
    pos = _lattice(basis, (reps,) * 3, a)
    pos = pos + _rng(seed).normal(0.0, sigma, pos.shape)
    num = np.full(len(pos), ATOMIC_NUMBERS["Si"], np.int64)
    return Structure(pos, num, np.eye(3) * a * reps, info={"config": "C1", "seed": seed})


def rocksalt(seed=2, reps=12, a=6.46, sigma=0.05, species=("Pb", "Te")):
    anion = [(x + 0.5, y, z) for x, y, z in FCC]
    pos = _lattice(FCC + anion, (reps,) * 3, a)
    num = np.tile(np.array([ATOMIC_NUMBERS[species[0]]] * 4 + [ATOMIC_NUMBERS[species[1]]] * 4),
                  reps ** 3)
    pos = pos + _rng(seed).normal(0.0, sigma, pos.shape)
    return Structure(pos, num.astype(np.int64), np.eye(3) * a * reps,
                     info={"config": "C2", "seed": seed, "species": species})


def fcc_alloy(seed=3, reps=17, a=3.6, sigma=0.1, species=("Cr", "Mn", "Fe", "Co", "Ni")):
    rng = _rng(seed)
    pos = _lattice(FCC, (reps,) * 3, a)
    n = len(pos)
    k = len(species)
    counts = [n // k + (1 if t < n % k else 0) for t in range(k)]
    labels = np.repeat(np.arange(k), counts)
    rng.shuffle(labels)
    num = np.array([ATOMIC_NUMBERS[species[t]] for t in labels], np.int64)
    pos = pos + rng.normal(0.0, sigma, pos.shape)
    return Structure(pos, num, np.eye(3) * a * reps,
                     info={"config": "C3", "seed": seed, "species": species})


def _rsa_cubic(rng, n, length, dmin, batch=65536):
    """Random sequential placement in a cubic periodic box (minimum image).

    Grid cells of side <= dmin/sqrt(3) hold at most one atom, so a candidate
    is checked against the cells within ``ceil(dmin/h)``.  Candidates are
    drawn in batches and tested in two vectorised steps: against atoms already
    placed, then against earlier candidates of the same batch (a candidate that
    conflicts with any earlier survivor is dropped, kept or not).  The result
    is a deterministic function of the seed.
    """
    g = int(math.floor(length / (dmin / math.sqrt(3.0))))
    h = length / g
    reach = int(math.ceil(dmin / h))
    occ = np.full((g, g, g), -1, np.int64)
    pos = np.empty((n, 3))
    count = 0
    offs = np.stack(np.meshgrid(*[np.arange(-reach, reach + 1)] * 3, indexing="ij"), -1).reshape(-1, 3)
    rounds = 0
    while count < n:
        rounds += 1
        if rounds > 5000:
            raise RuntimeError("random sequential placement did not converge")
        cand = rng.random((batch, 3)) * length
        cell = np.floor(cand / h).astype(np.int64) % g
        nbc = (cell[:, None, :] + offs[None, :, :]) % g
        who = occ[nbc[..., 0], nbc[..., 1], nbc[..., 2]]
        has = who >= 0
        d = cand[:, None, :] - pos[np.where(has, who, 0)]
        d -= length * np.round(d / length)
        ok = ~(has & ((d * d).sum(-1) < dmin * dmin)).any(axis=1)
        idx = np.nonzero(ok)[0]
        if idx.size == 0:
            continue
        # earlier survivors of this batch, lowest index per grid cell
        tmp = np.full((g, g, g), np.iinfo(np.int64).max, np.int64)
        cs = cell[idx]
        np.minimum.at(tmp, (cs[:, 0], cs[:, 1], cs[:, 2]), idx)
        nb = (cs[:, None, :] + offs[None, :, :]) % g
        other = tmp[nb[..., 0], nb[..., 1], nb[..., 2]]
        earlier = other < idx[:, None]
        d = cand[idx][:, None, :] - cand[np.where(earlier, other, 0)]
        d -= length * np.round(d / length)
        clash = (earlier & ((d * d).sum(-1) < dmin * dmin)).any(axis=1)
        same = tmp[cs[:, 0], cs[:, 1], cs[:, 2]] != idx
        keep = idx[~(clash | same)][: n - count]
        k = keep.size
        pos[count:count + k] = cand[keep]
        kc = cell[keep]
        occ[kc[:, 0], kc[:, 1], kc[:, 2]] = np.arange(count, count + k)
        count += k
    return pos


def amorphous(seed=4, n_atoms=100_000, density=0.08, dmin=1.8, n_species=10):
    rng = _rng(seed)
    length = (n_atoms / density) ** (1.0 / 3.0)
    species = tuple(rng.choice(OAM_ELEMENTS, size=n_species, replace=False))
    pos = _rsa_cubic(rng, n_atoms, length, dmin)
    labels = rng.integers(0, n_species, n_atoms)
    num = np.array([ATOMIC_NUMBERS[species[t]] for t in labels], np.int64)
    return Structure(pos, num, np.eye(3) * length,
                     info={"config": "C4", "seed": seed, "species": species})


def _random_triclinic(rng):
    while True:
        a, b, c = rng.uniform(4.0, 10.0, 3)
        al, be, ga = np.radians(rng.uniform(70.0, 110.0, 3))
        cx = c * math.cos(be)
        cy = c * (math.cos(al) - math.cos(be) * math.cos(ga)) / math.sin(ga)
        cz2 = c * c - cx * cx - cy * cy
        if cz2 <= 0.25 * c * c:          # reject near-singular cells
            continue
        cell = np.array([[a, 0.0, 0.0],
                         [b * math.cos(ga), b * math.sin(ga), 0.0],
                         [cx, cy, math.sqrt(cz2)]])
        return cell


def _rsa_all_images(rng, n, cell, dmin, max_rounds=50, batch=256):
    """Placement checking every periodic image (images within +-2 cells)."""
    images = np.stack(np.meshgrid(*[np.arange(-2, 3)] * 3, indexing="ij"), -1).reshape(-1, 3) @ cell
    pos = np.empty((0, 3))
    for _ in range(max_rounds):
        cand = rng.random((batch, 3)) @ cell
        for p in cand:
            if len(pos):
                d = p[None, None, :] - (pos[:, None, :] + images[None, :, :])
                if ((d * d).sum(-1) < dmin * dmin).any():
                    continue
            pos = np.vstack([pos, p])
            if len(pos) == n:
                return pos
    return None


def small_cells(seed=5, n_cells=256, dmin=1.8):
    rng = _rng(seed)
    out = []
    while len(out) < n_cells:
        n = int(rng.integers(8, 65))
        species = tuple(rng.choice(OAM_ELEMENTS, size=int(rng.integers(1, 5)), replace=False))
        pos = None
        while pos is None:
            cell = _random_triclinic(rng)
            th = abs(np.linalg.det(cell)) / np.array(
                [np.linalg.norm(np.cross(cell[(d + 1) % 3], cell[(d + 2) % 3])) for d in range(3)])
            # a cell denser than 0.09 atoms/Å^3 or thinner than dmin is redrawn
            if n / abs(np.linalg.det(cell)) > 0.09 or th.min() <= dmin:
                continue
            pos = _rsa_all_images(rng, n, cell, dmin)
        labels = rng.integers(0, len(species), n)
        num = np.array([ATOMIC_NUMBERS[species[t]] for t in labels], np.int64)
        out.append(Structure(pos, num, cell, info={"config": "C5", "index": len(out),
                                                   "species": species}))
    return out


CONFIGS = {
    "C1": ("mobius-oam-loc", si_diamond),
    "C2": ("nep-seeded", rocksalt),
    "C3": ("mobius-oam-mp", fcc_alloy),
    "C4": ("mobius-oam-eq", amorphous),
    "C5": ("mobius-oam-eq", small_cells),
}
