"""MI355X-native evaluator of RUNE's Möbius and NEP4 potentials.

Drop-in plugin modules: ``rune_amd.mobius.plugin`` and ``rune_amd.nep.plugin``
(same API as ``rune.mobius.plugin`` / ``rune.nep.plugin``).  Array API:
``rune_amd.api.Evaluator``.  C ABI: ``include/rune_hip.h``.
"""

__version__ = "0.1.0"

ASSETS = __import__("pathlib").Path(__file__).resolve().parent / "assets"
MODELS = {name: ASSETS / "models" / name / "model.pt"
          for name in ("mobius-oam-loc", "mobius-oam-mp", "mobius-oam-eq")}
