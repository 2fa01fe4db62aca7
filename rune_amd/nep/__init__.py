"""NEP4 on the HIP evaluator; drop-in for ``rune.nep``."""
