"""``BatchBuilder`` of ``rune/mobius/interface/batch.py:103-197`` (GPU neighbour lists)."""

from ...interface import BatchBuilder as _Builder


class BatchBuilder(_Builder):
    def __init__(self, params, device, dtype):
        super().__init__(params, device, dtype, kind="Möbius")


__all__ = ["BatchBuilder"]
