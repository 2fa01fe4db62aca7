"""Möbius (Local / MP / EQ) on the HIP evaluator; drop-in for ``rune.mobius``."""
