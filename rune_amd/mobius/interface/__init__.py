"""ASE interface of the Möbius plugin (``rune/mobius/interface``)."""
