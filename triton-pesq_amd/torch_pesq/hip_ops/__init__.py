"""HIP operators of the PESQ pipeline, one module per stage.

Mirrors the operator set of the reference's ``torch_pesq/triton_ops``:
``HipIIR`` (``TritonIIR``), ``HipResample`` (``TritonResample``),
``HipStftBark`` (``TritonStftBark``), ``HipPesqChain`` (``TritonPesqChain``),
the element-wise functions and ``PesqLossHip`` (``PesqLossTriton``).
"""

import torch

HAS_HIP = torch.cuda.is_available()

__all__ = ["HAS_HIP"]
