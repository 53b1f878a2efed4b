"""``torch_pesq.triton_ops.chain`` (``chain.py:68,1024``): ``TritonPesqChain`` is :class:`HipPesqChain`."""

from ..hip_ops.chain import HipPesqChain

TritonPesqChain = HipPesqChain

__all__ = ["TritonPesqChain"]
