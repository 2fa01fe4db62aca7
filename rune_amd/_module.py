"""``nn.Module`` shell shared by the Möbius and NEP drop-in models.

The shell holds parameters and buffers under the reference's state_dict
names (so ``load_state_dict(strict=True)`` accepts the reference
checkpoints), and its ``forward(batch)`` evaluates through the HIP library:
the padded reference batch (``rune/mobius/interface/batch.py:124-166``) is
converted to records on the HIP device and ``rune_model_compute`` returns
energies, forces and virials.  There is no PyTorch/CPU evaluation path: a
batch whose tensors live on the host is evaluated on the current HIP device
and the results come back on the batch's device.  The kernels compute in
float32; a float64 module (the reference keeps float64 checkpoints float64)
is evaluated with float32 copies of its weights and returns its own dtype.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import _native as N


class HipPotential(nn.Module):
    family = N.FAMILY_MOBIUS

    def __init__(self):
        super().__init__()
        self._native = None
        self._native_key = None
        self._nlist = None

    # the handle is rebuilt whenever a parameter or buffer changed in place
    def _state_key(self):
        return tuple((t.data_ptr(), t._version) for t in self.state_dict().values())

    def native(self):
        key = self._state_key()
        if self._native is None or key != self._native_key:
            # NativeModel hands the weights over as float32 copies
            self._native = N.NativeModel(self.params, self.state_dict(), self.family)
            self._native_key = key
        return self._native

    def neighbor_list(self):
        if self._nlist is None:
            self._nlist = N.NeighborList()
        return self._nlist

    def _direct_edge_list(self):
        return "angular" if self.family == N.FAMILY_NEP else "radial"

    def forward(self, batch):
        """``Mobius.forward`` / ``NEP.forward`` contract on a padded batch."""
        compute_forces = bool(batch.get("compute_forces", True))
        compute_virial = bool(batch.get("compute_virial", True))
        positions = batch["positions"]
        dev = N.compute_device(positions.device)
        to_dev = lambda t, dtype=None: t.detach().to(device=dev, dtype=dtype)
        counts = batch["n_atoms_per_structure"].detach().to("cpu", torch.long)
        struct_ptr = torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)]).numpy()
        nl = self.neighbor_list().from_padded(
            to_dev(positions, torch.float32), to_dev(batch["radial_neighbors"]),
            to_dev(batch["radial_offsets"], torch.float32), to_dev(batch["angular_neighbors"]),
            to_dev(batch["angular_offsets"], torch.float32), struct_ptr)
        out = self.native().compute(nl, to_dev(batch["types"]), len(struct_ptr) - 1,
                                    compute_forces, compute_virial)
        back = lambda t: t.to(device=positions.device, dtype=positions.dtype)
        result = {"energies": back(out["energies"]), "energy": back(out["energy"])}
        if compute_forces:
            result["forces"] = back(out["forces"])
        if compute_virial:
            result["virial"] = back(out["virial"])
        return result


class ParamHolder(nn.Module):
    """Bare module that only carries named parameters / buffers."""


def linear(n_in, n_out, bias=True):
    return nn.Linear(n_in, n_out, bias=bias)
