"""PESQ loss on AMD Instinct GPUs (gfx950), a drop-in for ``torch_pesq``.

``from torch_pesq import PesqLoss, PesqLossTriton`` gives the same classes as
the reference package (``torch_pesq/__init__.py:1-32``); both run on HIP
kernels.  ``PesqLossTriton`` (alias of ``PesqLossHip``) adds ``graphed()``.
"""

from .bark import *  # noqa: F401,F403
from .loudness import *  # noqa: F401,F403
from .loss import PesqLoss


def __getattr__(name):
    """Import the graph capable GPU class lazily, like the reference does."""

    if name in ("PesqLossTriton", "PesqLossHip"):
        from .hip_ops.loss import PesqLossHip

        return PesqLossHip
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")


__all__ = [
    "PesqLoss",
    "PesqLossTriton",
    "PesqLossHip",
    "BarkScale",
    "Loudness",
]
