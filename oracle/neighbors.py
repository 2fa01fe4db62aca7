"""CPU oracle for the directed periodic neighbour lists (numpy, fp64).

TEST INFRASTRUCTURE ONLY (see ``oracle/model.py``).

Restates ``rune/mobius/interface/batch.py:42-102`` (identical in
``rune/nep/interface/batch.py``): candidate pairs ``(i, j, S)`` from
``ase.neighborlist.neighbor_list("ijS", atoms, max(rc))`` (``batch.py:74``)
are kept when the fp64 test of ``batch.py:76-82`` passes:

    offset = S @ cell                       (fp64)
    vector = (p[j] + offset) - p[i]         (fp64)
    d2     = vector . vector
    radial  : d2 < rc_radial**2,   angular : d2 < rc_angular**2

ASE is not available, so the candidate set is enumerated here directly (every
image of every atom, self-pairs excluded at S = 0), and the arithmetic is
pinned to one evaluation order with no fused multiply-add:

    offset_d = (S0*c[0,d] + S1*c[1,d]) + S2*c[2,d]
    d2       = (v0*v0 + v1*v1) + v2*v2

For orthorhombic cells every order gives the same bits; for triclinic cells
the reference's BLAS matmul may differ from this in the last ulp (unpinned).

Order.  ASE's within-centre order is not pinned by any reference test.  The
canonical order used here and by the HIP builder: edges sorted by centre,
then by *class* (0 = inside both cutoffs, 1 = inside only the larger one),
then by neighbour index, then by the shift ``(S0, S1, S2)``.  The list of the
smaller cutoff is therefore a prefix of every centre's segment.

Vectors handed to the model are ``(fp32(p[j]) + fp32(offset)) - fp32(p[i])``
in fp32, the cast the reference performs in ``batch.py:146-163`` followed by
the subtraction of ``descriptor.py:813-817``.
"""

from __future__ import annotations

import numpy as np


class NeighborOverflow(ValueError):
    pass


def _thickness(cell):
    vol = abs(np.linalg.det(cell))
    out = np.empty(3)
    for d in range(3):
        a, b = cell[(d + 1) % 3], cell[(d + 2) % 3]
        out[d] = vol / np.linalg.norm(np.cross(a, b))
    return out


def offsets_of(shifts, cell):
    s = shifts.astype(np.float64)
    out = np.empty_like(s)
    for d in range(3):
        out[:, d] = (s[:, 0] * cell[0, d] + s[:, 1] * cell[1, d]) + s[:, 2] * cell[2, d]
    return out


def _d2(positions, i, j, off):
    v = (positions[j] + off) - positions[i]
    return (v[:, 0] * v[:, 0] + v[:, 1] * v[:, 1]) + v[:, 2] * v[:, 2]


def _candidates_bruteforce(positions, cell, pbc, rc):
    n = len(positions)
    th = _thickness(cell)
    inv = np.linalg.inv(cell)
    frac = positions @ inv
    span = frac.max(0) - frac.min(0) if n else np.zeros(3)
    rng = [np.arange(-(int(np.ceil(rc / th[d] + span[d])) + 1),
                     int(np.ceil(rc / th[d] + span[d])) + 2) if pbc[d] else np.zeros(1, np.int64)
           for d in range(3)]
    S = np.stack(np.meshgrid(*rng, indexing="ij"), -1).reshape(-1, 3).astype(np.int64)
    ii, jj = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
    ii, jj = ii.ravel(), jj.ravel()
    out_i, out_j, out_s = [], [], []
    for s in S:
        keep = ~((ii == jj) & (not s.any()))
        i, j = ii[keep], jj[keep]
        off = offsets_of(np.broadcast_to(s, (len(i), 3)), cell)
        m = _d2(positions, i, j, off) < rc * rc
        out_i.append(i[m]); out_j.append(j[m]); out_s.append(np.broadcast_to(s, (int(m.sum()), 3)))
    if not out_i:
        return np.zeros(0, np.int64), np.zeros(0, np.int64), np.zeros((0, 3), np.int64)
    return np.concatenate(out_i), np.concatenate(out_j), np.concatenate(out_s)


def _candidates_celllist(positions, cell, pbc, rc):
    """Cell-list enumeration with fractional bins of width >= rc."""
    n = len(positions)
    th = _thickness(cell)
    inv = np.linalg.inv(cell)
    frac = positions @ inv
    wrap = np.where(np.asarray(pbc)[None, :], np.floor(frac), 0.0).astype(np.int64)
    fw = frac - wrap
    nb = np.maximum(1, np.floor(th / (rc * (1.0 + 1e-9)))).astype(np.int64)
    lo = np.zeros(3, np.int64)
    nbins = nb.copy()
    b = np.floor(fw * nb).astype(np.int64)
    for d in range(3):
        if pbc[d]:
            b[:, d] = np.clip(b[:, d], 0, nb[d] - 1)
        else:
            lo[d] = b[:, d].min()
            nbins[d] = b[:, d].max() - lo[d] + 1
            b[:, d] -= lo[d]
    m = (np.floor(rc * nb / th) + 1).astype(np.int64)
    flat = (b[:, 0] * nbins[1] + b[:, 1]) * nbins[2] + b[:, 2]
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=int(np.prod(nbins)))
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]])
    out_i, out_j, out_s = [], [], []
    for dx in range(-m[0], m[0] + 1):
        for dy in range(-m[1], m[1] + 1):
            for dz in range(-m[2], m[2] + 1):
                nbb = b + np.array([dx, dy, dz])
                T = np.zeros_like(nbb)
                ok = np.ones(n, bool)
                for d in range(3):
                    if pbc[d]:
                        T[:, d] = np.floor_divide(nbb[:, d], nb[d])
                        nbb[:, d] = nbb[:, d] - T[:, d] * nb[d]
                    else:
                        ok &= (nbb[:, d] >= 0) & (nbb[:, d] < nbins[d])
                idx = np.nonzero(ok)[0]
                if idx.size == 0:
                    continue
                f2 = (nbb[idx, 0] * nbins[1] + nbb[idx, 1]) * nbins[2] + nbb[idx, 2]
                c = counts[f2]
                i = np.repeat(idx, c)
                base = np.repeat(starts[f2] - np.concatenate([[0], np.cumsum(c)[:-1]]), c)
                j = order[base + np.arange(c.sum())]
                S = np.repeat(T[idx], c, axis=0) - wrap[j] + wrap[i]
                keep = ~((i == j) & ~S.any(axis=1))
                i, j, S = i[keep], j[keep], S[keep]
                mask = _d2(positions, i, j, offsets_of(S, cell)) < rc * rc
                out_i.append(i[mask]); out_j.append(j[mask]); out_s.append(S[mask])
    if not out_i:
        return np.zeros(0, np.int64), np.zeros(0, np.int64), np.zeros((0, 3), np.int64)
    return np.concatenate(out_i), np.concatenate(out_j), np.concatenate(out_s)


def effective_cell(positions, cell, pbc):
    """Replace degenerate non-periodic cell rows by spanning vectors.

    Non-periodic directions always carry ``S_d = 0``, so their cell row only
    shapes the binning.  A zero row (a molecule without a cell) is replaced by
    an orthogonal vector longer than the atoms' extent.
    """
    cell = np.array(cell, dtype=np.float64).reshape(3, 3)
    for d in range(3):
        if not pbc[d] and np.linalg.norm(cell[d]) == 0.0:
            extent = np.ptp(positions, axis=0).max() if len(positions) else 0.0
            cell[d] = 0.0
            cell[d, d] = extent + 10.0
    if abs(np.linalg.det(cell)) < 1e-12:
        raise ValueError("cell is singular in a periodic direction")
    return cell


def build(positions, cell, pbc, rc_radial, rc_angular, *, max_radial=None, max_angular=None,
          method="auto"):
    """Return the canonical CSR neighbour lists of one structure.

    Result dict (numpy): ``ptr[N+1]`` over the union (larger-cutoff) list,
    ``n_short[N]`` edges of the smaller cutoff per centre (segment prefix),
    ``center, neighbor[E]``, ``shift[E,3]`` int, ``offset[E,3]`` fp64,
    ``d2[E]`` fp64, ``vec32[E,3]`` fp32, ``radial_mask, angular_mask[E]``.
    """
    positions = np.ascontiguousarray(positions, dtype=np.float64)
    pbc = [bool(x) for x in np.broadcast_to(np.asarray(pbc, bool), (3,))]
    n = len(positions)
    rc = max(rc_radial, rc_angular)
    cell_eff = effective_cell(positions, cell, pbc)
    if n == 0:
        i = j = np.zeros(0, np.int64)
        S = np.zeros((0, 3), np.int64)
    else:
        th = _thickness(cell_eff)
        use_brute = method == "brute" or (method == "auto" and n <= 64)
        if use_brute:
            i, j, S = _candidates_bruteforce(positions, cell_eff, pbc, rc)
        else:
            i, j, S = _candidates_celllist(positions, cell_eff, pbc, rc)
        del th
    off = offsets_of(S, cell_eff) if len(S) else np.zeros((0, 3))
    d2 = _d2(positions, i, j, off) if len(i) else np.zeros(0)
    rmask = d2 < rc_radial * rc_radial
    amask = d2 < rc_angular * rc_angular
    short_mask = amask if rc_angular <= rc_radial else rmask
    cls = (~short_mask).astype(np.int64)
    order = np.lexsort((S[:, 2], S[:, 1], S[:, 0], j, cls, i)) if len(i) else np.zeros(0, np.int64)
    i, j, S, off, d2 = i[order], j[order], S[order], off[order], d2[order]
    rmask, amask, short_mask = rmask[order], amask[order], short_mask[order]
    counts = np.bincount(i, minlength=n) if n else np.zeros(0, np.int64)
    ptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    n_short = np.bincount(i[short_mask], minlength=n) if n else np.zeros(0, np.int64)
    for name, mask, cap in (("radial", rmask, max_radial), ("angular", amask, max_angular)):
        if cap is None or n == 0:
            continue
        c = np.bincount(i[mask], minlength=n)
        if c.max(initial=0) > cap:
            atom = int(np.argmax(c))
            raise NeighborOverflow(
                f"Neighbor count {int(c.max())} for atom {atom} exceeds "
                f"max_neighbors={cap}. Increase max_neighbors_radial "
                "or max_neighbors_angular.")
    p32 = positions.astype(np.float32)
    vec32 = (p32[j] + off.astype(np.float32)) - p32[i]
    return {
        "ptr": ptr, "n_short": n_short.astype(np.int64), "center": i, "neighbor": j,
        "shift": S, "offset": off, "d2": d2, "vec32": vec32.astype(np.float32),
        "radial_mask": rmask, "angular_mask": amask, "cell": cell_eff,
    }


def split(nl):
    """Radial and angular edge lists ``(center, neighbor, offset)`` from :func:`build`."""
    out = {}
    for name in ("radial", "angular"):
        m = nl[f"{name}_mask"]
        out[name] = (nl["center"][m], nl["neighbor"][m], nl["offset"][m])
    return out


def pack(center, neighbor, offsets, n_atoms, max_neighbors):
    """Padded ``[N, max]`` arrays with -1 padding, ``batch.py:9-39``."""
    nb = np.full((n_atoms, max_neighbors), -1, dtype=np.int64)
    of = np.zeros((n_atoms, max_neighbors, 3), dtype=np.float64)
    if center.size == 0:
        return nb, of
    order = np.argsort(center, kind="stable")
    center, neighbor, offsets = center[order], neighbor[order], offsets[order]
    counts = np.bincount(center, minlength=n_atoms)
    if counts.max() > max_neighbors:
        atom = int(np.argmax(counts))
        raise NeighborOverflow(
            f"Neighbor count {int(counts.max())} for atom {atom} exceeds "
            f"max_neighbors={max_neighbors}. Increase max_neighbors_radial "
            "or max_neighbors_angular.")
    starts = np.cumsum(counts) - counts
    slots = np.arange(center.size) - np.repeat(starts, counts)
    nb[center, slots] = neighbor
    of[center, slots] = offsets
    return nb, of
