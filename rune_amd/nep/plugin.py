"""NEP4 plugin API, drop-in for ``rune.nep.plugin`` (``rune/nep/plugin.py``).

Same names and behaviour: ``PLUGIN_NAME``, ``resolve_params`` (GPUMD limits,
``:100-228``), ``build_model``, ``get_ddp_options``, ``load_model`` (accepts
``*.txt``, ``:57-75``), ``export_model`` (``:78-85``) and
``build_calculator``.  Checkpoints are read with ``weights_only=True``.
"""

from __future__ import annotations

from math import isfinite
from pathlib import Path
from typing import Any, Mapping

import torch

from ..elements import ATOMIC_NUMBERS
from .model import NEP

PLUGIN_NAME = "nep4"

_DESCRIPTOR_DEFAULTS: dict[str, Any] = {
    "rcut_radial": 8.0, "rcut_angular": 4.0, "n_max_radial": 4, "n_max_angular": 4,
    "basis_size_radial": 8, "basis_size_angular": 8, "l_max": 4, "l_max_4body": 2,
    "l_max_5body": 0, "has_q_112": 0, "has_q_123": 0, "has_q_233": 0, "has_q_134": 0,
    "max_neighbors_radial": 100, "max_neighbors_angular": 30, "zbl": None,
}

_INTEGER_RANGES = {
    "n_max_radial": (0, 12), "n_max_angular": (0, 8), "basis_size_radial": (0, 16),
    "basis_size_angular": (0, 12), "l_max": (2, 8),
}
_HIGHER_ORDER = ("l_max_4body", "l_max_5body", "has_q_112", "has_q_123", "has_q_233",
                 "has_q_134")


def _is_int(v):
    return isinstance(v, int) and not isinstance(v, bool)


def _copy(value):
    if isinstance(value, dict):
        return {k: _copy(v) for k, v in value.items()}
    if isinstance(value, list):
        return [_copy(v) for v in value]
    return value


def _resolve_descriptor(params: Mapping[str, Any], extra_defaults: Mapping[str, Any]):
    if not isinstance(params, Mapping):
        raise TypeError("Model params must be a TOML table.")
    defaults = {**_DESCRIPTOR_DEFAULTS, **dict(extra_defaults)}
    unknown = sorted(set(params) - set(defaults) - {"elements"})
    if unknown:
        raise ValueError(f"Unknown model parameter(s): {', '.join(unknown)}")
    if "elements" not in params:
        raise ValueError('Model params must define elements = ["..."].')
    v = {**defaults, **dict(params)}
    els = v["elements"]
    if not isinstance(els, list) or not els or not all(isinstance(e, str) for e in els):
        raise ValueError("elements must be a non-empty list of chemical symbols.")
    if len(set(els)) != len(els):
        raise ValueError("elements must not contain duplicates.")
    if len(els) > 94:
        raise ValueError("GPUMD supports at most 94 elements (H through Pu).")
    bad = [e for e in els if e not in ATOMIC_NUMBERS or e == "X"]
    if bad:
        raise ValueError(f"Unknown chemical element symbols: {bad}.")
    unsupported = [e for e in els if not 1 <= ATOMIC_NUMBERS[e] <= 94]
    if unsupported:
        raise ValueError(f"GPUMD supports elements H through Pu; unsupported: {unsupported}.")
    for name in ("rcut_radial", "rcut_angular"):
        x = v[name]
        if not isinstance(x, (int, float)) or isinstance(x, bool) or not isfinite(x):
            raise ValueError(f"{name} must be a finite number.")
    if not 3.0 <= v["rcut_angular"] <= v["rcut_radial"] <= 100.0:
        raise ValueError("NEP cutoffs must satisfy 3 <= rcut_angular <= rcut_radial <= 100 Å.")
    for name, (lo, hi) in _INTEGER_RANGES.items():
        if not _is_int(v[name]) or not lo <= v[name] <= hi:
            raise ValueError(f"{name} must be an integer in [{lo}, {hi}].")
    for name in _HIGHER_ORDER:
        allowed = (0, 2) if name == "l_max_4body" else (0, 1)
        if not _is_int(v[name]) or v[name] not in allowed:
            raise ValueError(f"{name} must be one of {allowed}.")
    if (v["has_q_123"] or v["has_q_233"]) and v["l_max"] < 3:
        raise ValueError("q_123 and q_233 require l_max >= 3.")
    if v["has_q_134"] and v["l_max"] < 4:
        raise ValueError("q_134 requires l_max >= 4.")
    channels = v["l_max"] + sum(v[n] > 0 for n in _HIGHER_ORDER)
    if (v["n_max_angular"] + 1) * channels > 90:
        raise ValueError("The number of angular descriptors must not exceed 90.")
    for name in ("max_neighbors_radial", "max_neighbors_angular"):
        if not _is_int(v[name]) or v[name] < 1:
            raise ValueError(f"{name} must be a positive integer.")
    out = {
        "elements": list(els), "rcut_radial": float(v["rcut_radial"]),
        "rcut_angular": float(v["rcut_angular"]), "n_desc_radial": int(v["n_max_radial"]) + 1,
        "n_desc_angular": int(v["n_max_angular"]) + 1,
        "k_max_radial": int(v["basis_size_radial"]) + 1,
        "k_max_angular": int(v["basis_size_angular"]) + 1, "l_max": int(v["l_max"]),
        "l_max_4body": int(v["l_max_4body"]), "l_max_5body": int(v["l_max_5body"]),
        "has_q_222": int(int(v["l_max_4body"]) > 0), "has_q_1111": int(int(v["l_max_5body"]) > 0),
        "has_q_112": int(int(v["has_q_112"]) > 0), "has_q_123": int(int(v["has_q_123"]) > 0),
        "has_q_233": int(int(v["has_q_233"]) > 0), "has_q_134": int(int(v["has_q_134"]) > 0),
        "max_neighbors_radial": int(v["max_neighbors_radial"]),
        "max_neighbors_angular": int(v["max_neighbors_angular"]), "n_types": len(els),
    }
    for name in extra_defaults:
        out[name] = _copy(v[name])
    if v["zbl"] is not None:
        out["zbl"] = _copy(v["zbl"])
    return out


def resolve_params(values: dict) -> dict:
    resolved = _resolve_descriptor(values, {"hidden_dims": [30]})
    hd = resolved["hidden_dims"]
    if not isinstance(hd, list) or len(hd) != 1 or not _is_int(hd[0]) or not 1 <= hd[0] <= 200:
        raise ValueError(
            "NEP hidden_dims must contain exactly one positive integer in [1, 200]. "
            "RUNE currently supports single-hidden-layer NEP models for GPUMD export.")
    resolved["hidden_dims"] = list(hd)
    return resolved


def build_model(params: dict):
    return NEP(params)


def get_ddp_options(params: dict) -> dict:
    return {"find_unused_parameters": True}


def load_model(path, device=None):
    path = Path(path)
    if path.suffix.lower() == ".txt":
        return NEP.from_nep_txt(path, device=device)
    ck = torch.load(path, map_location="cpu", weights_only=True)
    identity = ck.get("plugin")
    if not isinstance(identity, dict) or identity.get("name") != PLUGIN_NAME:
        raise ValueError(f"Checkpoint is not a {PLUGIN_NAME} model: {path}")
    params = ck.get("model_params")
    if not isinstance(params, dict):
        raise ValueError(f"Checkpoint does not contain resolved model_params: {path}")
    model = NEP(params)
    name, _ = next(model.named_parameters())
    model.to(dtype=ck["model_state_dict"][name].dtype)
    model.load_state_dict(ck["model_state_dict"], strict=True)
    if device is not None:
        model.to(device)
    return model


def export_model(model, path):
    path = Path(path)
    if path.name == "model":
        path = path.with_name("nep.txt")
    elif path.name.startswith("model_epoch_"):
        path = path.with_name(path.name.replace("model_", "nep_") + ".txt")
    model.save_nep_txt(path)
    return path


def build_calculator(artifact, **kwargs):
    from .interface.calculator import Calculator
    return Calculator(artifact, **kwargs)
