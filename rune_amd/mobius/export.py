"""``mobius1`` text export, format of ``rune/mobius/export.py:79-146`` unchanged.

Layout: header ``mobius1 <T> <elements>``, ``schema 1``, ``ints K`` + K
``name value`` lines, ``reals K`` (``%.17g``), ``tensors K`` with ``name ndim
dims`` and the values 8 per line (``%.17g``), then ``END``.  Tensors are the
state_dict (as float64, so float32 weights round-trip bit for bit) followed by
the sparse angular-polynomial table (``desc.basis_terms/offsets``), the sparse
invariant table (``desc.invariant_terms/offsets``) and the orthonormal scale.
"""

from __future__ import annotations

import math
from math import comb
from pathlib import Path

import torch

from .. import tables as T


def complex_power_terms(power, imaginary):
    """(coefficient, x power, y power) of Re / Im of (x + i y)^power."""
    out = []
    for yp in range(power + 1):
        if imaginary:
            if yp % 2 == 0:
                continue
            sign = -1.0 if ((yp - 1) // 2) % 2 else 1.0
        else:
            if yp % 2:
                continue
            sign = -1.0 if (yp // 2) % 2 else 1.0
        out.append((sign * comb(power, yp), power - yp, yp))
    return out


def basis_terms(angular):
    """Rows [component, coefficient, x, y, z powers] of every real angular polynomial."""
    rows, offsets, comp = [], [0], 0
    for L in range(1, angular.L_max + 1):
        zc = getattr(angular, f"Z{L}").detach().cpu().double()
        for n1 in range(L + 1):
            for imaginary in ([False] if n1 == 0 else [False, True]):
                for xy, xp, yp in complex_power_terms(n1, imaginary):
                    for zp in range((L + n1) % 2, L - n1 + 1, 2):
                        coefficient = xy * zc[n1, zp].item()
                        if coefficient:
                            rows.append([comp, coefficient, xp, yp, zp])
                comp += 1
                offsets.append(len(rows))
    return torch.tensor(rows, dtype=torch.float64), torch.tensor(offsets, dtype=torch.float64)


def invariant_terms(angular):
    """Rows [output, coefficient, degree, i0..i3] of every invariant polynomial."""
    channels = []
    c3 = angular.C3B.detach().cpu().double().tolist()
    for L in range(1, angular.L_max + 1):
        a, b = L * L - 1, (L + 1) ** 2 - 1
        channels.append([(c3[k] * (1 if k == a else 2), (k, k)) for k in range(a, b)])
    if angular.has_q_222:
        c = angular.C4B.detach().cpu().double().tolist()
        channels.append([(c[0], (3, 3, 3)), (c[1], (3, 4, 4)), (c[1], (3, 5, 5)),
                         (c[2], (3, 6, 6)), (c[2], (3, 7, 7)), (c[3], (6, 5, 5)),
                         (-c[3], (6, 4, 4)), (c[4], (4, 5, 7))])
    if angular.has_q_1111:
        c = angular.C5B.detach().cpu().double().tolist()
        channels.append([(c[0], (0, 0, 0, 0)), (c[1], (0, 0, 1, 1)), (c[1], (0, 0, 2, 2)),
                         (c[2], (1, 1, 1, 1)), (2 * c[2], (1, 1, 2, 2)), (c[2], (2, 2, 2, 2))])
    if angular.has_q_112:
        c = angular.C4B2.detach().cpu().double().tolist()
        channels.append([(c[0], (0, 0, 3)), (c[1], (0, 1, 4)), (c[1], (0, 2, 5)),
                         (c[2], (3, 1, 1)), (c[2], (3, 2, 2)), (c[3], (6, 1, 1)),
                         (-c[3], (6, 2, 2)), (c[4], (1, 2, 7))])
    for enabled, terms in ((angular.has_q_123, T.Q123_TERMS), (angular.has_q_233, T.Q233_TERMS),
                           (angular.has_q_134, T.Q134_TERMS)):
        if enabled:
            channels.append(terms)
    rows, offsets = [], [0]
    for out, terms in enumerate(channels):
        for coefficient, idx in terms:
            rows.append([out, coefficient, len(idx), *idx, *([-1] * (4 - len(idx)))])
        offsets.append(len(rows))
    return torch.tensor(rows, dtype=torch.float64), torch.tensor(offsets, dtype=torch.float64)


def orthonormal_scale(l_max):
    """sqrt(2 C3B), halved inside the root at m = 0, in float64."""
    size = l_max * (l_max + 2)
    metric = torch.tensor(T.C3B[:size], dtype=torch.float64) * 2.0
    for L in range(1, l_max + 1):
        metric[L * L - 1] *= 0.5
    return metric.sqrt()


def export_data(model):
    if any(v.dtype not in (torch.float32, torch.float64) for v in model.state_dict().values()):
        raise ValueError("Native Möbius export requires float32 or float64 weights and buffers.")
    p = model.params
    names = ("n_desc_radial", "n_desc_angular", "k_max_radial", "k_max_angular", "l_max",
             "hidden_dim", "blocks", "ffn_dim", "message_layers", "message_dim", "pair_dim",
             "message_groups", "vector_channels", "message_basis_size", "max_neighbors_radial",
             "max_neighbors_angular")
    ints = {n: int(p[n]) for n in names}
    acts = {"tanh": 0, "silu": 1, "swish": 1, "gelu": 2}
    ints.update(n_types=model.n_elements, num_L=model.num_L, input_dim=model.input_dim,
                message_mode=int(model.message_mode == "equivariant"),
                equivariant_channels=model.equivariant_channels,
                equivariant_l_max=model.equivariant_l_max,
                activation=acts[model.activation.strip().lower()],
                zbl_enabled=int(model.zbl is not None),
                zbl_flexible=int(model.zbl is not None and model.zbl.flexible))
    reals = {n: float(p[n]) for n in ("rcut_radial", "rcut_angular", "message_cutoff", "norm_eps")}
    reals.update(zbl_rc_inner=model.zbl.rc_inner if model.zbl else 0.0,
                 zbl_rc_outer=model.zbl.rc_outer if model.zbl else 0.0)
    if not all(math.isfinite(v) for v in reals.values()):
        raise ValueError("Cannot export nonfinite Möbius configuration values.")
    tensors = {k: v.detach().cpu().double().contiguous() for k, v in model.state_dict().items()}
    ang = model.descriptor.angular
    tensors["desc.basis_terms"], tensors["desc.basis_offsets"] = basis_terms(ang)
    tensors["desc.invariant_terms"], tensors["desc.invariant_offsets"] = invariant_terms(ang)
    tensors["desc.orthonormal_scale"] = orthonormal_scale(ang.L_max)
    if not all(torch.isfinite(v).all() for v in tensors.values()):
        raise ValueError("Cannot export a Möbius model containing nonfinite values.")
    return ints, reals, tensors


def export_model(model, path):
    """Write ``mobius.txt`` and return its path (naming of ``export.py:120-128``)."""
    path = Path(path)
    if path.name == "model":
        path = path.with_name("mobius.txt")
    elif path.name.startswith("model_epoch_"):
        path = path.with_name(path.name.replace("model_", "mobius_", 1) + ".txt")
    ints, reals, tensors = export_data(model)
    path.parent.mkdir(parents=True, exist_ok=True)
    with path.open("w", encoding="utf-8", newline="\n") as fh:
        fh.write(f"mobius1 {model.n_elements} {' '.join(model.elements)}\n")
        fh.write("schema 1\n")
        fh.write(f"ints {len(ints)}\n")
        for k, v in ints.items():
            fh.write(f"{k} {v}\n")
        fh.write(f"reals {len(reals)}\n")
        for k, v in reals.items():
            fh.write(f"{k} {v:.17g}\n")
        fh.write(f"tensors {len(tensors)}\n")
        for k, v in tensors.items():
            fh.write(f"{k} {v.ndim} {' '.join(str(s) for s in v.shape)}\n")
            flat = v.reshape(-1).tolist()
            for s in range(0, len(flat), 8):
                fh.write(" ".join(format(x, ".17g") for x in flat[s:s + 8]) + "\n")
        fh.write("END\n")
    return path


def read_mobius_txt(path):
    """Parse a ``mobius1`` file into (elements, ints, reals, tensors as float64)."""
    with open(path, encoding="utf-8") as fh:
        tokens = fh.read().split("\n")
    it = iter(tokens)
    head = next(it).split()
    if head[0] != "mobius1":
        raise ValueError("not a mobius1 file")
    elements = head[2:2 + int(head[1])]
    if next(it).split() != ["schema", "1"]:
        raise ValueError("unsupported schema")
    ints, reals, tensors = {}, {}, {}
    n = int(next(it).split()[1])
    for _ in range(n):
        k, v = next(it).split()
        ints[k] = int(v)
    n = int(next(it).split()[1])
    for _ in range(n):
        k, v = next(it).split()
        reals[k] = float(v)
    n = int(next(it).split()[1])
    for _ in range(n):
        parts = next(it).split()
        name, ndim = parts[0], int(parts[1])
        dims = [int(x) for x in parts[2:2 + ndim]]
        count = 1
        for d in dims:
            count *= d
        vals = []
        while len(vals) < count:
            vals.extend(float(x) for x in next(it).split())
        tensors[name] = torch.tensor(vals, dtype=torch.float64).reshape(dims)
    if next(it).strip() != "END":
        raise ValueError("missing END")
    return elements, ints, reals, tensors
