"""Descriptor parameter/buffer shell with the reference's state_dict layout.

``rune/mobius/descriptor.py:443-555`` (identical in ``rune/nep``): the radial
and angular coefficient tables ``c_table[t_i, t_j, n, k]`` are parameters
initialised with ``randn``; C3B, C4B, C5B, C4B2 and Z1..Z8 are persistent
float32 buffers.  The evaluation itself runs in the HIP kernels.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import tables as T


class RadialDescriptor(nn.Module):
    def __init__(self, n_types, n_desc, k_max, r_c):
        super().__init__()
        self.n_types, self.n_desc, self.k_max, self.r_c = n_types, n_desc, k_max, r_c
        self.c_table = nn.Parameter(torch.randn(n_types, n_types, n_desc, k_max))


class AngularDescriptor(nn.Module):
    def __init__(self, n_types, n_desc, k_max, r_c, l_max, flags):
        super().__init__()
        self.n_types, self.n_desc, self.k_max, self.r_c = n_types, n_desc, k_max, r_c
        self.L_max = l_max
        (self.has_q_222, self.has_q_1111, self.has_q_112, self.has_q_123, self.has_q_233,
         self.has_q_134) = flags
        if (self.has_q_123 or self.has_q_233) and l_max < 3:
            raise ValueError("q_123 and q_233 require l_max >= 3.")
        if self.has_q_134 and l_max < 4:
            raise ValueError("q_134 requires l_max >= 4.")
        self.num_L = l_max + sum(flags)
        self.c_table = nn.Parameter(torch.randn(n_types, n_types, n_desc, k_max))
        self.register_buffer("C3B", torch.tensor(T.C3B, dtype=torch.float32))
        self.register_buffer("C4B", torch.tensor(T.C4B, dtype=torch.float32))
        self.register_buffer("C5B", torch.tensor(T.C5B, dtype=torch.float32))
        self.register_buffer("C4B2", torch.tensor(T.C4B2, dtype=torch.float32))
        for L in range(1, 9):
            self.register_buffer(f"Z{L}", torch.tensor(T.Z_COEFF[L], dtype=torch.float32))

    def orthonormal_scale(self, reference, l_max):
        """``descriptor.py:626-637``: sqrt(2 C3B), halved at m = 0, in ``reference``'s dtype."""
        size = l_max * (l_max + 2)
        metric = reference.new_tensor(T.C3B[:size]) * 2.0
        for order in range(1, l_max + 1):
            metric[order * order - 1] *= 0.5
        return metric.sqrt()


def descriptor_flags(params):
    """(q222, q1111, q112, q123, q233, q134) as ``descriptor.py:893-900`` resolves them."""
    return (
        int(params.get("has_q_222", int(params.get("l_max_4body", 2) > 0)) > 0),
        int(params.get("has_q_1111", int(params.get("l_max_5body", 0) > 0)) > 0),
        int(int(params.get("has_q_112", 0)) > 0),
        int(int(params.get("has_q_123", 0)) > 0),
        int(int(params.get("has_q_233", 0)) > 0),
        int(int(params.get("has_q_134", 0)) > 0),
    )


class Descriptor(nn.Module):
    def __init__(self, params):
        super().__init__()
        self.radial = RadialDescriptor(params["n_types"], params["n_desc_radial"],
                                       params["k_max_radial"], params["rcut_radial"])
        flags = descriptor_flags(params)
        self.angular = AngularDescriptor(params["n_types"], params["n_desc_angular"],
                                         params["k_max_angular"], params["rcut_angular"],
                                         params["l_max"], flags)
        params["l_max_4body"] = 2 if flags[0] else 0
        params["l_max_5body"] = flags[1]
        for name, value in zip(("has_q_222", "has_q_1111", "has_q_112", "has_q_123",
                                "has_q_233", "has_q_134"), flags):
            params[name] = value


class ZBLBuffers(nn.Module):
    """Buffers of ``ZBLRepulsion`` (``rune/mobius/zbl.py:24-67``)."""

    def __init__(self, elements, config, atomic_numbers):
        super().__init__()
        if isinstance(config, dict):
            inner, outer = float(config["rc_inner"]), float(config["rc_outer"])
            flexible = bool(config.get("flexible", inner == 0.0 and outer == 0.0))
            parameters = config.get("parameters")
        else:
            if len(config) != 2:
                raise ValueError("zbl must be [rc_inner, rc_outer] or a mapping.")
            inner, outer = map(float, config)
            flexible = inner == 0.0 and outer == 0.0
            parameters = None
        if flexible and parameters is None:
            raise ValueError("Flexible ZBL requires ten parameters per element pair.")
        if not flexible and not (0.0 <= inner < outer):
            raise ValueError("Universal ZBL requires 0 <= rc_inner < rc_outer.")
        self.rc_inner, self.rc_outer, self.flexible = inner, outer, flexible
        n = len(elements)
        self.register_buffer("atomic_numbers", torch.tensor(
            [atomic_numbers[e] for e in elements], dtype=torch.float32))
        self.register_buffer("universal_coefficients",
                             torch.tensor(T.UNIVERSAL_ZBL, dtype=torch.float32))
        if flexible:
            tensor = torch.as_tensor(parameters, dtype=torch.float32).reshape(-1, 10)
            if tensor.shape[0] != n * (n + 1) // 2:
                raise ValueError(f"Flexible ZBL expects {n * (n + 1) // 2} pair rows, "
                                 f"got {tensor.shape[0]}.")
            if not torch.isfinite(tensor).all():
                raise ValueError("Flexible ZBL parameters must all be finite.")
            if ((tensor[:, 0] < 0.0) | (tensor[:, 0] >= tensor[:, 1])).any():
                raise ValueError("Each flexible ZBL pair must satisfy 0 <= rc_inner < rc_outer.")
        else:
            tensor = torch.zeros((0, 10), dtype=torch.float32)
        self.register_buffer("pair_parameters", tensor)
        self.max_rc_outer = float(tensor[:, 1].max()) if flexible else outer
