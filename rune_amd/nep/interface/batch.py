"""``BatchBuilder`` of ``rune/nep/interface/batch.py:103-197`` (GPU neighbour lists)."""

from ...interface import BatchBuilder as _Builder


class BatchBuilder(_Builder):
    def __init__(self, params, device, dtype):
        super().__init__(params, device, dtype, kind="NEP")


__all__ = ["BatchBuilder"]
