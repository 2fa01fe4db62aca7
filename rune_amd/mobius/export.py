"""Writer and reader of the ``mobius1`` text artifact.

The byte layout is the format of ``rune/mobius/export.py:79-146`` (read by
``rune/mobius/src/mobius.cu:26-151``) and does not change: a header line
``mobius1 <T> <elements>``, ``schema 1``, three sections -- ``ints K``,
``reals K`` and ``tensors K`` -- whose entries are listed in a fixed order,
then ``END``.  Reals and tensor values are printed with 17 significant
digits (``%.17g``), tensor values eight to a line, so float32 weights
promoted to float64 round-trip bit for bit.  The tensors are the state_dict
followed by four descriptor tables the native reader evaluates directly: the
real angular polynomials as sparse monomial rows, the invariant polynomials
as sparse product rows, and the orthonormal direction metric.

Here the section contents are declared as data (``_INT_FIELDS``,
``_REAL_FIELDS``), the angular table is obtained by expanding
``Z_L[|m|](z) * Re/Im (x + i y)^|m|`` with a small sparse-polynomial
product, and the invariant table is generated from the term groups in
``rune_amd.tables``.
"""

from __future__ import annotations

import math
from pathlib import Path

import torch

from .. import tables as T

_ACTIVATION_CODES = {"tanh": 0, "silu": 1, "swish": 1, "gelu": 2}

# ints section: (name, value of a model); the order is part of the format
_INT_FIELDS = tuple((name, (lambda n: lambda m: int(m.params[n]))(name)) for name in (
    "n_desc_radial", "n_desc_angular", "k_max_radial", "k_max_angular", "l_max", "hidden_dim",
    "blocks", "ffn_dim", "message_layers", "message_dim", "pair_dim", "message_groups",
    "vector_channels", "message_basis_size", "max_neighbors_radial", "max_neighbors_angular")) + (
    ("n_types", lambda m: m.n_elements),
    ("num_L", lambda m: m.num_L),
    ("input_dim", lambda m: m.input_dim),
    ("message_mode", lambda m: int(m.message_mode == "equivariant")),
    ("equivariant_channels", lambda m: m.equivariant_channels),
    ("equivariant_l_max", lambda m: m.equivariant_l_max),
    ("activation", lambda m: _ACTIVATION_CODES[m.activation.strip().lower()]),
    ("zbl_enabled", lambda m: int(m.zbl is not None)),
    ("zbl_flexible", lambda m: int(m.zbl is not None and m.zbl.flexible)),
)

# reals section
_REAL_FIELDS = tuple((name, (lambda n: lambda m: float(m.params[n]))(name)) for name in (
    "rcut_radial", "rcut_angular", "message_cutoff", "norm_eps")) + (
    ("zbl_rc_inner", lambda m: m.zbl.rc_inner if m.zbl else 0.0),
    ("zbl_rc_outer", lambda m: m.zbl.rc_outer if m.zbl else 0.0),
)


# -- sparse polynomials in x, y: {(x power, y power): integer coefficient} --

def _times_variable(poly, axis):
    return {(xp + (axis == 0), yp + (axis == 1)): c for (xp, yp), c in poly.items()}


def _add(a, b, sign=1):
    out = dict(a)
    for key, c in b.items():
        out[key] = out.get(key, 0) + sign * c
    return {k: c for k, c in out.items() if c != 0}


def _complex_power(n):
    """Real and imaginary parts of (x + i y)^n as integer-coefficient polynomials."""
    re, im = {(0, 0): 1}, {}
    for _ in range(n):
        re, im = (_add(_times_variable(re, 0), _times_variable(im, 1), -1),
                  _add(_times_variable(re, 1), _times_variable(im, 0)))
    return re, im


def angular_polynomials(angular):
    """Sparse rows ``[component, coefficient, x power, y power, z power]`` of
    every real angular basis function up to ``L_max`` and the row offsets per
    component.  Component order per order L: |m| = 0, then (Re, Im) for
    |m| = 1..L; rows within a component by ascending y power, then z power
    (``rune/mobius/descriptor.py:574-624``)."""
    rows, offsets = [], [0]
    component = 0
    for order in range(1, angular.L_max + 1):
        z_table = getattr(angular, f"Z{order}").detach().cpu().double()
        for m in range(order + 1):
            re, im = _complex_power(m)
            for part in ((re,) if m == 0 else (re, im)):
                z_powers = range((order + m) % 2, order - m + 1, 2)
                for (xp, yp), xy in sorted(part.items(), key=lambda kv: kv[0][1]):
                    for zp in z_powers:
                        value = float(xy) * z_table[m, zp].item()
                        if value != 0.0:
                            rows.append([component, value, xp, yp, zp])
                component += 1
                offsets.append(len(rows))
    return torch.tensor(rows, dtype=torch.float64), torch.tensor(offsets, dtype=torch.float64)


def _grouped(coefficients, groups):
    return [(mult * coefficients[index], idx) for index, terms in groups for mult, idx in terms]


def invariant_polynomials(angular):
    """Sparse rows ``[output, coefficient, degree, i0, i1, i2, i3]`` (unused
    indices -1) of the invariant polynomials q of one radial channel, in the
    output order L = 1..L_max, q222, q1111, q112, q123, q233, q134
    (``rune/mobius/descriptor.py:650-733``), and the row offsets per output."""
    buffer = lambda name: getattr(angular, name).detach().cpu().double().tolist()
    c3 = buffer("C3B")
    outputs = []
    for order in range(1, angular.L_max + 1):
        first = order * order - 1
        outputs.append([(c3[k] * (1.0 if k == first else 2.0), (k, k))
                        for k in range(first, first + 2 * order + 1)])
    optional = ((angular.has_q_222, lambda: _grouped(buffer("C4B"), T.Q222_GROUPS)),
                (angular.has_q_1111, lambda: _grouped(buffer("C5B"), T.Q1111_GROUPS)),
                (angular.has_q_112, lambda: _grouped(buffer("C4B2"), T.Q112_GROUPS)),
                (angular.has_q_123, lambda: T.Q123_TERMS),
                (angular.has_q_233, lambda: T.Q233_TERMS),
                (angular.has_q_134, lambda: T.Q134_TERMS))
    outputs += [terms() for enabled, terms in optional if enabled]
    rows, offsets = [], [0]
    for out, terms in enumerate(outputs):
        rows += [[out, coefficient, len(idx)] + list(idx) + [-1] * (4 - len(idx))
                 for coefficient, idx in terms]
        offsets.append(len(rows))
    return torch.tensor(rows, dtype=torch.float64), torch.tensor(offsets, dtype=torch.float64)


def direction_metric(l_max):
    """Orthonormal scale sqrt(2 C3B), with the m = 0 entries sqrt(C3B), in float64
    from the decimal constants (``rune/mobius/descriptor.py:626-637``)."""
    size = l_max * (l_max + 2)
    m0 = {order * order - 1 for order in range(1, l_max + 1)}
    return torch.tensor([math.sqrt(T.C3B[k] * (1.0 if k in m0 else 2.0)) for k in range(size)],
                        dtype=torch.float64)


def export_data(model):
    """(ints, reals, tensors) of the artifact, checked for finiteness."""
    state = model.state_dict()
    if any(v.dtype not in (torch.float32, torch.float64) for v in state.values()):
        raise ValueError("Native Möbius export requires float32 or float64 weights and buffers.")
    ints = {name: get(model) for name, get in _INT_FIELDS}
    reals = {name: get(model) for name, get in _REAL_FIELDS}
    if not all(math.isfinite(v) for v in reals.values()):
        raise ValueError("Cannot export nonfinite Möbius configuration values.")
    tensors = {k: v.detach().cpu().double().contiguous() for k, v in state.items()}
    angular = model.descriptor.angular
    tensors["desc.basis_terms"], tensors["desc.basis_offsets"] = angular_polynomials(angular)
    tensors["desc.invariant_terms"], tensors["desc.invariant_offsets"] = \
        invariant_polynomials(angular)
    tensors["desc.orthonormal_scale"] = direction_metric(angular.L_max)
    if not all(bool(torch.isfinite(v).all()) for v in tensors.values()):
        raise ValueError("Cannot export a Möbius model containing nonfinite values.")
    return ints, reals, tensors


def _text(model, ints, reals, tensors):
    lines = [f"mobius1 {model.n_elements} {' '.join(model.elements)}", "schema 1",
             f"ints {len(ints)}"]
    lines += [f"{k} {v}" for k, v in ints.items()]
    lines.append(f"reals {len(reals)}")
    lines += [f"{k} {v:.17g}" for k, v in reals.items()]
    lines.append(f"tensors {len(tensors)}")
    for name, value in tensors.items():
        lines.append(" ".join([name, str(value.ndim)] + [str(d) for d in value.shape]))
        flat = [format(x, ".17g") for x in value.reshape(-1).tolist()]
        lines += [" ".join(flat[i:i + 8]) for i in range(0, len(flat), 8)]
    lines.append("END")
    return "\n".join(lines) + "\n"


def artifact_path(path):
    """``model`` -> ``mobius.txt``; ``model_epoch_<k>`` -> ``mobius_epoch_<k>.txt``
    (the checkpoint-to-artifact naming of ``rune/mobius/export.py:120-128``)."""
    path = Path(path)
    if path.name == "model":
        return path.with_name("mobius.txt")
    if path.name.startswith("model_epoch_"):
        return path.with_name("mobius" + path.name[len("model"):] + ".txt")
    return path


def export_model(model, path):
    """Write the ``mobius1`` artifact of ``model`` and return its path."""
    path = artifact_path(path)
    text = _text(model, *export_data(model))
    path.parent.mkdir(parents=True, exist_ok=True)
    with path.open("w", encoding="utf-8", newline="\n") as fh:
        fh.write(text)
    return path


def read_mobius_txt(path):
    """Parse a ``mobius1`` file into (elements, ints, reals, tensors as float64)."""
    with open(path, encoding="utf-8") as fh:
        lines = iter(fh.read().split("\n"))
    head = next(lines).split()
    if not head or head[0] != "mobius1":
        raise ValueError("not a mobius1 file")
    elements = head[2:2 + int(head[1])]
    if next(lines).split() != ["schema", "1"]:
        raise ValueError("unsupported schema")

    def section(label):
        word, count = next(lines).split()
        if word != label:
            raise ValueError(f"expected the {label} section")
        return int(count)

    ints = dict((k, int(v)) for k, v in (next(lines).split() for _ in range(section("ints"))))
    reals = dict((k, float(v)) for k, v in (next(lines).split() for _ in range(section("reals"))))
    tensors = {}
    for _ in range(section("tensors")):
        name, ndim, *dims = next(lines).split()
        shape = [int(d) for d in dims[:int(ndim)]]
        values = []
        while len(values) < math.prod(shape):
            values += [float(x) for x in next(lines).split()]
        tensors[name] = torch.tensor(values, dtype=torch.float64).reshape(shape)
    if next(lines).strip() != "END":
        raise ValueError("missing END")
    return elements, ints, reals, tensors
