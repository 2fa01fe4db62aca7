"""ASE ``Calculator`` of ``rune/nep/interface/calculator.py`` on the HIP evaluator."""

from ...interface import make_calculator_class
from ..plugin import load_model

Calculator = make_calculator_class(load_model, "NEP")

__all__ = ["Calculator"]
