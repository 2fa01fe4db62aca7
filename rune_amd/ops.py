"""PyTorch custom-op registration of the HIP evaluator.

``torch.ops.rune_hip.evaluate(handle, positions, types, struct_ptr, cells, pbc,
compute_forces, compute_virial)`` runs the neighbour search and the E + F +
virial evaluation of a registered evaluator on the current HIP stream and
returns ``(energies[N], energy[B], forces[N,3], virial[B,9])`` (forces /
virial are empty when not requested).  The op is a thin shell over the C ABI
(``include/rune_hip.h``); PyTorch only supplies memory and the stream.
"""

from __future__ import annotations

import itertools
import weakref

import torch

_HANDLES: dict[int, weakref.ref] = {}
_NEXT = itertools.count(1)


def register(evaluator) -> int:
    """Handle for ``evaluator``; the registry holds a weak reference only."""
    handle = next(_NEXT)
    _HANDLES[handle] = weakref.ref(evaluator)
    return handle


def unregister(handle: int) -> None:
    _HANDLES.pop(handle, None)


@torch.library.custom_op("rune_hip::evaluate", mutates_args=())
def evaluate(handle: int, positions: torch.Tensor, types: torch.Tensor, struct_ptr: list[int],
             cells: list[float], pbc: list[int], compute_forces: bool,
             compute_virial: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                                            torch.Tensor]:
    ev = _HANDLES[handle]()
    if ev is None:
        raise RuntimeError(f"rune_hip evaluator handle {handle} is no longer alive")
    p = ev.params
    nb = len(struct_ptr) - 1
    ev.nlist.build(positions, struct_ptr, cells, pbc, p["rcut_radial"], p["rcut_angular"],
                   p["max_neighbors_radial"], p["max_neighbors_angular"])
    out = ev.native.compute(ev.nlist, types, nb, compute_forces, compute_virial)
    dev = positions.device
    forces = out.get("forces", torch.empty((0, 3), dtype=torch.float32, device=dev))
    virial = out.get("virial", torch.empty((0, 9), dtype=torch.float32, device=dev))
    return out["energies"], out["energy"], forces, virial


@evaluate.register_fake
def _(handle, positions, types, struct_ptr, cells, pbc, compute_forces, compute_virial):
    n, nb = positions.shape[0], len(struct_ptr) - 1
    f = positions.new_empty((n if compute_forces else 0, 3), dtype=torch.float32)
    v = positions.new_empty((nb if compute_virial else 0, 9), dtype=torch.float32)
    return (positions.new_empty(n, dtype=torch.float32),
            positions.new_empty(nb, dtype=torch.float32), f, v)
