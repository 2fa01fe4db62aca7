"""Möbius plugin API, drop-in for ``rune.mobius.plugin`` (``rune/mobius/plugin.py``).

``PLUGIN_NAME``, ``resolve_params`` (``:53-114``, ``:157-239``),
``build_model``, ``get_ddp_options``, ``load_model`` (``:125-142``),
``build_calculator`` (``:145-148``) and ``export_model`` (``:151-154``) keep
their names, arguments and errors.  Checkpoints load with
``torch.load(weights_only=True)``.
"""

from __future__ import annotations

from pathlib import Path
from typing import Any, Mapping

import torch

from ..elements import ATOMIC_NUMBERS
from .model import Mobius

PLUGIN_NAME = "mobius-force-field"

_DESCRIPTOR_DEFAULTS: dict[str, Any] = {
    "rcut_radial": 8.0, "rcut_angular": 4.0, "n_max_radial": 4, "n_max_angular": 4,
    "basis_size_radial": 8, "basis_size_angular": 8, "l_max": 4, "l_max_4body": 2,
    "l_max_5body": 0, "has_q_112": 0, "has_q_123": 0, "has_q_233": 0, "has_q_134": 0,
    "max_neighbors_radial": 100, "max_neighbors_angular": 30, "zbl": None,
}

_DEFAULTS = {
    "hidden_dim": 96, "blocks": 3, "ffn_dim": 192, "activation": "silu", "message_layers": 2,
    "message_dim": 64, "pair_dim": 16, "message_groups": 8, "vector_channels": 8,
    "message_basis_size": None, "message_cutoff": None, "message_mode": "scalar",
    "equivariant_channels": 8, "equivariant_l_max": None, "norm_eps": 1.0e-8,
}


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
    bad = [e for e in els if e not in ATOMIC_NUMBERS or e == "X"]
    if bad:
        raise ValueError(f"Unknown chemical element symbols: {bad}.")
    for name in ("rcut_radial", "rcut_angular"):
        x = v[name]
        if not isinstance(x, (int, float)) or isinstance(x, bool) or x <= 0:
            raise ValueError(f"{name} must be positive.")
    for name in ("n_max_radial", "n_max_angular", "basis_size_radial", "basis_size_angular",
                 "l_max", "max_neighbors_radial", "max_neighbors_angular"):
        if not _is_int(v[name]) or v[name] < 1:
            raise ValueError(f"{name} must be a positive integer.")
    if v["l_max"] > 8:
        raise ValueError("l_max must be in 1..8.")
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
    r = _resolve_descriptor(values, _DEFAULTS)
    for name in ("hidden_dim", "ffn_dim", "message_dim", "pair_dim", "message_groups"):
        if not _is_int(r[name]) or r[name] < 1:
            raise ValueError(f"{name} must be a positive integer.")
    for name in ("blocks", "message_layers", "vector_channels"):
        if not _is_int(r[name]) or r[name] < 0:
            raise ValueError(f"{name} must be a nonnegative integer.")
    if r["message_mode"] not in ("scalar", "equivariant"):
        raise ValueError("message_mode must be 'scalar' or 'equivariant'.")
    if r["message_mode"] == "equivariant":
        ch, order = r["equivariant_channels"], r["equivariant_l_max"]
        if order is None:
            order = r["l_max"]
        if not _is_int(ch) or ch < 1:
            raise ValueError("equivariant_channels must be a positive integer.")
        if not _is_int(order) or not 1 <= order <= min(r["l_max"], 8):
            raise ValueError("equivariant_l_max must be in 1..min(l_max, 8).")
        if r["message_layers"] < 1:
            raise ValueError("equivariant message_mode requires message_layers >= 1.")
        r["equivariant_l_max"] = order
    else:
        if "equivariant_channels" in values or "equivariant_l_max" in values:
            raise ValueError("Equivariant parameters require message_mode='equivariant'.")
        for name in ("message_mode", "equivariant_channels", "equivariant_l_max"):
            r.pop(name)
    if r["hidden_dim"] % r["message_groups"] != 0:
        raise ValueError("hidden_dim must be divisible by message_groups.")
    if r["message_basis_size"] is None:
        r["message_basis_size"] = r["k_max_radial"]
    if not _is_int(r["message_basis_size"]) or r["message_basis_size"] < 1:
        raise ValueError("message_basis_size must be a positive integer.")
    if r["message_cutoff"] is None:
        r["message_cutoff"] = r["rcut_radial"]
    if not 0.0 < float(r["message_cutoff"]) <= r["rcut_radial"]:
        raise ValueError("message_cutoff must be positive and cannot exceed rcut_radial.")
    r["message_cutoff"] = float(r["message_cutoff"])
    if not isinstance(r["activation"], str) or not r["activation"]:
        raise ValueError("activation must be a non-empty string.")
    if not isinstance(r["norm_eps"], (int, float)) or r["norm_eps"] <= 0:
        raise ValueError("norm_eps must be positive.")
    r["norm_eps"] = float(r["norm_eps"])
    return r


def build_model(params: dict):
    return Mobius(params)


def get_ddp_options(params: dict) -> dict:
    return {"find_unused_parameters": False}


def load_model(path, device=None):
    path = Path(path)
    ck = torch.load(path, map_location="cpu", weights_only=True)
    identity = ck.get("plugin")
    if not isinstance(identity, dict) or identity.get("name") != PLUGIN_NAME:
        raise ValueError(f"Checkpoint is not a {PLUGIN_NAME} model: {path}")
    params = ck.get("model_params")
    if not isinstance(params, dict):
        raise ValueError(f"Checkpoint does not contain resolved model_params: {path}")
    model = Mobius(params)
    name, _ = next(model.named_parameters())
    model.to(dtype=ck["model_state_dict"][name].dtype)
    model.load_state_dict(ck["model_state_dict"], strict=True)
    if device is not None:
        model.to(device)
    return model


def build_calculator(artifact, **kwargs):
    from .interface.calculator import Calculator
    return Calculator(artifact, **kwargs)


def export_model(model, path):
    from .export import export_model as write_model
    return write_model(model, path)
