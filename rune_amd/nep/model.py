"""NEP4 drop-in model: reference state_dict layout, ``nep.txt`` I/O, HIP forward.

Mirrors ``rune/nep/model.py``: ``NEP(params)`` (:49-85) with per-element
``element_mlps[element] = Sequential(Linear(Q, H), Tanh(), Linear(H, 1,
bias=False))``, the ``q_scaler`` buffer, optional ZBL buffers and the
``shared_bias`` parameter; ``from_nep_txt`` (:284-489) and ``save_nep_txt``
(:491-579) keep the GPUMD text format unchanged.  ``forward(batch)`` runs on
the HIP device (energies ``E_i = w1.tanh(W0 (q*s) + b0) - shared_bias``,
``:157-170``; ZBL and the direct edge term on the angular list, ``:93``).
"""

from __future__ import annotations

import re

import torch
import torch.nn as nn

from .. import _native as N
from .._module import HipPotential
from ..descriptor import Descriptor, ZBLBuffers
from ..elements import ATOMIC_NUMBERS


class NEP(HipPotential):
    family = N.FAMILY_NEP
    model_family = "nep"

    def __init__(self, params):
        super().__init__()
        self.params = dict(params)
        self.descriptor = Descriptor(self.params)
        p = self.params
        self.n_desc_radial = p["n_desc_radial"]
        self.n_desc_angular = p["n_desc_angular"]
        self.L_max = p["l_max"]
        self.num_L = self.descriptor.angular.num_L
        (self.has_q_222, self.has_q_1111, self.has_q_112, self.has_q_123, self.has_q_233,
         self.has_q_134) = (self.descriptor.angular.has_q_222, self.descriptor.angular.has_q_1111,
                            self.descriptor.angular.has_q_112, self.descriptor.angular.has_q_123,
                            self.descriptor.angular.has_q_233, self.descriptor.angular.has_q_134)
        self.elements = list(p["elements"])
        self.n_elements = len(self.elements)
        input_dim = self.n_desc_radial + self.n_desc_angular * self.num_L
        hidden = p["hidden_dims"]
        if len(hidden) != 1:
            raise ValueError("RUNE NEP models have exactly one hidden layer.")
        self.element_mlps = nn.ModuleDict()
        for element in self.elements:
            self.element_mlps[element] = nn.Sequential(
                nn.Linear(input_dim, hidden[0]), nn.Tanh(), nn.Linear(hidden[0], 1, bias=False))
        self.register_buffer("q_scaler", torch.ones(input_dim, dtype=torch.float32))
        self._configure_zbl()
        self.shared_bias = nn.Parameter(torch.zeros(1))

    def _configure_zbl(self):
        zbl = self.params.get("zbl")
        if zbl is None:
            self.zbl = None
            return
        self.zbl = ZBLBuffers(self.elements, zbl, ATOMIC_NUMBERS)
        if not self.zbl.max_rc_outer <= self.params["rcut_angular"]:
            raise ValueError("ZBL rc_outer cannot exceed rcut_angular because NEP "
                             "evaluates ZBL on the angular neighbor list.")

    # ---- nep.txt -------------------------------------------------------------

    @classmethod
    def from_nep_txt(cls, filepath, device=None):
        """Reader of ``rune/nep/model.py:284-489`` semantics (same checks and errors)."""
        with open(filepath) as fh:
            lines = [ln.strip() for ln in fh if ln.strip() != ""]
        idx = 0
        tokens = lines[idx].split()
        idx += 1
        m = re.fullmatch(r"nep(\d+)(?:_(.*))?", tokens[0].lower())
        if m is None:
            raise ValueError("Invalid nep.txt: first line should start with nep4 or nep5.")
        if int(m.group(1)) != 4:
            raise NotImplementedError("Only nep4 is supported by the RUNE loader.")
        has_zbl = "zbl" in (m.group(2) or "").split("_")
        num_types = int(tokens[1])
        elements = tokens[2:]
        if len(elements) != num_types:
            raise ValueError("Invalid nep.txt: element count mismatch.")
        zbl = None
        if has_zbl:
            tokens = lines[idx].split()
            idx += 1
            if tokens[0] != "zbl" or len(tokens) not in (3, 4):
                raise ValueError("Invalid nep.txt: zbl line not found after nep4_zbl header.")
            zbl = {"rc_inner": float(tokens[1]), "rc_outer": float(tokens[2]),
                   "flexible": float(tokens[1]) == 0.0 and float(tokens[2]) == 0.0}
            if len(tokens) == 4:
                raise NotImplementedError("Typewise ZBL cutoffs are not supported in RUNE.")
        tokens = lines[idx].split()
        idx += 1
        if tokens[0] != "cutoff":
            raise ValueError("Invalid nep.txt: cutoff line not found.")
        if len(tokens) == 5:
            rc_r, rc_a = float(tokens[1]), float(tokens[2])
            mn_r, mn_a = int(tokens[3]), int(tokens[4])
        else:
            if len(tokens) != num_types * 2 + 3:
                raise ValueError("Invalid nep.txt: cutoff line length mismatch.")
            rr = [float(tokens[1 + 2 * i]) for i in range(num_types)]
            ra = [float(tokens[2 + 2 * i]) for i in range(num_types)]
            if len(set(rr)) != 1 or len(set(ra)) != 1:
                raise NotImplementedError("Per-type cutoffs are not supported in RUNE.")
            rc_r, rc_a = rr[0], ra[0]
            mn_r, mn_a = int(tokens[-2]), int(tokens[-1])

        def keyed(key):
            nonlocal idx
            t = lines[idx].split()
            idx += 1
            if t[0] != key:
                raise ValueError(f"Invalid nep.txt: {key} line not found.")
            return t

        t = keyed("n_max")
        n_r, n_a = int(t[1]), int(t[2])
        t = keyed("basis_size")
        b_r, b_a = int(t[1]), int(t[2])
        t = keyed("l_max")
        lv = [int(v) for v in t[1:]]
        if not 1 <= len(lv) <= 7:
            raise ValueError("Invalid nep.txt: l_max should contain 1 to 7 values.")
        lv.extend([1, 0, 0, 0, 0, 0][len(lv) - 1:])
        l_max, q222, q1111, q112, q123, q233, q134 = lv
        t = lines[idx].split()
        idx += 1
        if t[0] != "ANN" or len(t) != 3:
            raise ValueError("Invalid nep.txt: expected ANN width 0.")
        hidden = int(t[1])
        if not 1 <= hidden <= 200:
            raise ValueError("Invalid nep.txt: ANN width must be in [1, 200].")
        if int(t[2]) != 0:
            raise ValueError(
                "RUNE only supports single-hidden-layer NEP text models (ANN width 0).")
        params = {
            "elements": elements, "rcut_radial": rc_r, "rcut_angular": rc_a,
            "n_desc_radial": n_r + 1, "n_desc_angular": n_a + 1,
            "k_max_radial": b_r + 1, "k_max_angular": b_a + 1, "l_max": l_max,
            "l_max_4body": 2 if q222 > 0 else 0, "l_max_5body": 1 if q1111 > 0 else 0,
            "has_q_222": int(q222 > 0), "has_q_1111": int(q1111 > 0), "has_q_112": int(q112 > 0),
            "has_q_123": int(q123 > 0), "has_q_233": int(q233 > 0), "has_q_134": int(q134 > 0),
            "max_neighbors_radial": mn_r, "max_neighbors_angular": mn_a,
            "hidden_dims": [hidden], "n_types": num_types,
        }
        if zbl is not None and not zbl["flexible"]:
            params["zbl"] = zbl
        model = cls(params)
        dim = params["n_desc_radial"] + params["n_desc_angular"] * model.num_L
        values = [float(v) for line in lines[idx:] for v in line.split()]
        pos = 0

        def take(n):
            nonlocal pos
            if pos + n > len(values):
                raise ValueError("Invalid nep.txt: not enough parameters.")
            out = torch.tensor(values[pos:pos + n], dtype=torch.float32)
            pos += n
            return out

        with torch.no_grad():
            for el in elements:
                mlp = model.element_mlps[el]
                mlp[0].weight.copy_(take(hidden * dim).reshape(hidden, dim))
                mlp[0].bias.copy_(-take(hidden))
                mlp[2].weight.copy_(take(hidden).view(1, -1))
            model.shared_bias.copy_(take(1))
            T = num_types
            for table, nd, kk in ((model.descriptor.radial.c_table, n_r + 1, b_r + 1),
                                  (model.descriptor.angular.c_table, n_a + 1, b_a + 1)):
                # file order: n, k, t1, t2 (rune/nep/model.py:455-470)
                flat = take(nd * kk * T * T).reshape(nd, kk, T, T)
                table.copy_(flat.permute(2, 3, 0, 1))
            model.q_scaler.copy_(take(dim))
            if zbl is not None and zbl["flexible"]:
                zbl["parameters"] = values[pos:]
                pos = len(values)
                model.params["zbl"] = zbl
                model._configure_zbl()
        if device is not None:
            model.to(device)
        return model

    def save_nep_txt(self, filepath):
        """Writer of ``rune/nep/model.py:491-579`` (``%18.10e`` values)."""
        p = self.params
        if len(p["hidden_dims"]) != 1:
            raise ValueError("RUNE nep.txt export requires exactly one NEP hidden layer.")
        if p["max_neighbors_radial"] > 819:
            raise ValueError("GPUMD nep.txt export requires max_neighbors_radial <= 819.")
        with open(filepath, "w") as f:
            zbl = self.zbl
            f.write(f"{'nep4_zbl' if zbl is not None else 'nep4'} {len(self.elements)} "
                    + " ".join(self.elements) + "\n")
            if zbl is not None:
                f.write(f"zbl {zbl.rc_inner} {zbl.rc_outer}\n")
            f.write(f"cutoff {p['rcut_radial']} {p['rcut_angular']} "
                    f"{p['max_neighbors_radial']} {p['max_neighbors_angular']}\n")
            f.write(f"n_max {int(p['n_desc_radial']) - 1} {int(p['n_desc_angular']) - 1}\n")
            f.write(f"basis_size {int(p['k_max_radial']) - 1} {int(p['k_max_angular']) - 1}\n")
            lv = [int(self.L_max), 2 if self.has_q_222 else 0, self.has_q_1111, self.has_q_112,
                  self.has_q_123, self.has_q_233, self.has_q_134]
            while len(lv) > 3 and lv[-1] == 0:
                lv.pop()
            f.write("l_max " + " ".join(str(v) for v in lv) + "\n")
            f.write(f"ANN {int(p['hidden_dims'][0])} 0\n")

            def put(values):
                for v in values:
                    f.write(f"{v:18.10e}\n")

            for el in self.elements:
                mlp = self.element_mlps[el]
                put(mlp[0].weight.detach().cpu().flatten().tolist())
                put((-mlp[0].bias.detach().cpu()).flatten().tolist())
                put(mlp[2].weight.detach().cpu().flatten().tolist())
            put([self.shared_bias.detach().cpu().item()])
            for table in (self.descriptor.radial.c_table, self.descriptor.angular.c_table):
                put(table.detach().cpu().permute(2, 3, 0, 1).flatten().tolist())
            put(self.q_scaler.detach().cpu().reshape(-1).tolist())
            if zbl is not None and zbl.flexible:
                put(zbl.pair_parameters.detach().cpu().reshape(-1).tolist())


def seeded_nep(seed=0, elements=("Pb", "Te"), n_max=(4, 4), basis=(8, 8), l_max=4,
               l_max_4body=2, l_max_5body=0, rcut=(6.0, 4.0), hidden=30,
               max_neighbors=(100, 30)):
    """Random-initialised NEP4 of the C2 configuration (``torch.manual_seed(seed)``)."""
    from .plugin import resolve_params
    params = resolve_params({
        "elements": list(elements), "n_max_radial": n_max[0], "n_max_angular": n_max[1],
        "basis_size_radial": basis[0], "basis_size_angular": basis[1], "l_max": l_max,
        "l_max_4body": l_max_4body, "l_max_5body": l_max_5body, "rcut_radial": rcut[0],
        "rcut_angular": rcut[1], "hidden_dims": [hidden],
        "max_neighbors_radial": max_neighbors[0], "max_neighbors_angular": max_neighbors[1],
    })
    torch.manual_seed(seed)
    return NEP(params)
