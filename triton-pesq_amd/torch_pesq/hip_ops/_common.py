"""Input validation shared by the HIP operators.

Mirrors the conventions of ``torch_pesq/triton_ops/_common.py:40-52`` of the
reference: inputs must live on a GPU and be float32, and are made contiguous.
"""

import torch

from .. import _lib

__all__ = ["check_input", "require_hip"]


def require_hip() -> None:
    """Raise a descriptive error when no GPU or no HIP library is available."""

    if not torch.cuda.is_available():
        raise RuntimeError("The HIP backend needs a ROCm GPU, none is visible.")
    _lib.library()


def check_input(tensor: torch.Tensor, name: str = "input") -> torch.Tensor:
    """Validate an operator input and return a contiguous GPU view of it."""

    if not isinstance(tensor, torch.Tensor):
        raise RuntimeError(f"`{name}` has to be a tensor, got {type(tensor).__name__}.")
    if not tensor.is_cuda:
        raise RuntimeError(f"The HIP backend needs `{name}` to live on a GPU.")
    if tensor.dtype != torch.float32:
        raise RuntimeError(f"The HIP backend only supports float32, `{name}` is {tensor.dtype}.")
    _lib.library()  # a GPU tensor means a visible GPU; this loads (once) the HIP library
    return tensor.contiguous()
