"""``torch_pesq.triton_ops.loss`` (``loss.py:15-18``): ``PesqLossTriton`` is :class:`PesqLossHip`."""

from ..hip_ops.loss import PesqLossTriton

__all__ = ["PesqLossTriton"]
