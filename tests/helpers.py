"""Helpers shared by the tests: weights, golden fixtures, oracle edge lists."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

from oracle import model as OM

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"


def load_weights(name, dtype=torch.float64):
    ck = torch.load(ROOT / f"rune_amd/assets/models/mobius-oam-{name}/model.pt",
                    weights_only=True, map_location="cpu")
    sd = {k: (v.to(dtype) if v.is_floating_point() else v)
          for k, v in ck["model_state_dict"].items()}
    return ck["model_params"], sd


def golden(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def edges_from(rec, kind, dtype=torch.float64):
    return OM.Edges(torch.as_tensor(rec[f"{kind}_center"]),
                    torch.as_tensor(rec[f"{kind}_neighbor"]),
                    torch.as_tensor(rec[f"{kind}_offset"], dtype=dtype))
