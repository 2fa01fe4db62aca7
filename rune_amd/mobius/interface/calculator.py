"""ASE ``Calculator`` of ``rune/mobius/interface/calculator.py`` on the HIP evaluator."""

from ...interface import make_calculator_class
from ..plugin import load_model

Calculator = make_calculator_class(load_model, "Möbius")

__all__ = ["Calculator"]
