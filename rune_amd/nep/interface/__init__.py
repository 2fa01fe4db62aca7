"""ASE interface of the NEP plugin (``rune/nep/interface``)."""
