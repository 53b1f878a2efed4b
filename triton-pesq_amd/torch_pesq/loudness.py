"""P.862 hearing thresholds and the Zwicker loudness module.

The threshold table, ``zwicker_power`` and ``Sl_16k`` are the P.862 constants
of ``torch_pesq/loudness.py:10-25`` in the reference, reproduced unchanged and
pinned by a CPU test against ``tests/golden/tables.json``.  :class:`Loudness`
keeps the attributes and methods of ``torch_pesq/loudness.py:28-129``.
"""

import torch
from torch.nn import Parameter

from .bark import centre_of_band_bark_16k, interp

__all__ = ["abs_thresh_power_16k", "zwicker_power", "Sl_16k", "Loudness"]

# fmt: off
abs_thresh_power_16k = [
    51286152.000000, 2454709.500000, 70794.593750, 4897.788574, 1174.897705,
    389.045166, 104.712860, 45.708820, 17.782795, 9.772372, 4.897789,
    3.090296, 1.905461, 1.258925, 0.977237, 0.724436, 0.562341, 0.457088,
    0.389045, 0.331131, 0.295121, 0.269153, 0.257040, 0.251189, 0.251189,
    0.251189, 0.251189, 0.263027, 0.288403, 0.309030, 0.338844, 0.371535,
    0.398107, 0.436516, 0.467735, 0.489779, 0.501187, 0.501187, 0.512861,
    0.524807, 0.524807, 0.524807, 0.512861, 0.478630, 0.426580, 0.371535,
    0.363078, 0.416869, 0.537032,
]
# fmt: on

zwicker_power = 0.23
Sl_16k = 1.866055e-001


def loudness_exponents() -> torch.Tensor:
    """Per band Zwicker exponents, evaluated in float32 exactly as P.862 tables do.

    ``(clamp(6 / (centre_bark + 2), 1, 2)) ** 0.15 * zwicker_power``; the
    centre table enters as a float32 tensor (``torch.tensor`` of a float list),
    so the exponents are float32 values (``torch_pesq/loudness.py:52-55``).
    """

    exp = 6 / (torch.tensor(centre_of_band_bark_16k) + 2.0)
    return exp.clamp(min=1.0, max=2.0) ** 0.15 * zwicker_power


class Loudness(torch.nn.Module):
    """Hearing thresholds and loudness curve per Bark band.

    Attributes
    ----------
    threshs : Parameter
        float64 hearing thresholds with shape ``[1, 1, nbark]``
    exp : Parameter
        float32 loudness exponents with shape ``[nbark]``
    """

    def __init__(self, nbark: int = 49):
        super().__init__()

        self.threshs = Parameter(
            interp(abs_thresh_power_16k, nbark).unsqueeze(0).unsqueeze(0),
            requires_grad=False,
        )
        self.exp = Parameter(loudness_exponents(), requires_grad=False)

    def total_audible(self, tensor: torch.Tensor, factor: float = 1.0) -> torch.Tensor:
        """Energy above ``factor`` times the threshold, summed over bands."""

        return (tensor * (tensor > self.threshs * factor)).sum(dim=2)

    def time_avg_audible(self, tensor: torch.Tensor, silent: torch.Tensor) -> torch.Tensor:
        """Mean over all frames of the audible (``> 100 th``), non silent energy."""

        mask = (tensor > self.threshs * 100.0) * (~silent.unsqueeze(2))
        return (tensor * mask).mean(dim=1)

    def forward(self, pow_dens: torch.Tensor) -> torch.Tensor:
        """Zwicker loudness, zero at or below the hearing threshold."""

        loudness = (2.0 * self.threshs) ** self.exp * (
            (0.5 + 0.5 * pow_dens / self.threshs) ** self.exp - 1
        )
        loudness = torch.where(pow_dens <= self.threshs, torch.zeros_like(loudness), loudness)
        return loudness * Sl_16k
