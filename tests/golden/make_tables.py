"""Write ``tables.json``: the literal constant tables of the reference as data.

Run in the build container only (the reference tree is not present on the GPU
box); the JSON it writes is committed and is what every test loads.

Sources, parsed as text (nothing from the reference is imported or executed):

* ``torch_pesq/bark.py:11-78``   Bark band tables and ``Sp_16k``
* ``torch_pesq/loudness.py:10-25`` hearing thresholds, ``zwicker_power``, ``Sl_16k``
* ``torch_pesq/loss.py:102-108`` pre-emphasis coefficients
* ``torch_pesq/triton_ops/loss.py`` / ``reference.py:322`` loudness constant ``sl``
"""

import json
import re
import sys
from pathlib import Path

REF = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
OUT = Path(__file__).with_name("tables.json")


def _list(text, name):
    match = re.search(name + r"\s*=\s*\[(.*?)\]", text, re.S)
    if match is None:
        raise SystemExit(f"table {name} not found")
    return [float(tok) for tok in re.findall(r"[-+0-9.eE]+", match.group(1))]


def _scalar(text, name):
    match = re.search(r"^" + name + r"\s*=\s*([-+0-9.eE]+)", text, re.M)
    if match is None:
        raise SystemExit(f"scalar {name} not found")
    return float(match.group(1))


def main():
    bark = (REF / "torch_pesq/bark.py").read_text()
    loud = (REF / "torch_pesq/loudness.py").read_text()
    loss = (REF / "torch_pesq/loss.py").read_text()

    pre = re.search(r"torch\.tensor\(\s*\[\[(.*?)\],\s*\[(.*?)\]\]", loss, re.S)

    tables = {
        "nr_of_hz_bands_per_bark_band_16k": [
            int(v) for v in _list(bark, "nr_of_hz_bands_per_bark_band_16k")
        ],
        "centre_of_band_bark_16k": _list(bark, "centre_of_band_bark_16k"),
        "centre_of_band_hz_16k": _list(bark, "centre_of_band_hz_16k"),
        "width_of_band_bark_16k": _list(bark, "width_of_band_bark_16k"),
        "width_of_band_hz_16k": _list(bark, "width_of_band_hz_16k"),
        "pow_dens_correction_factor_16k": _list(bark, "pow_dens_correction_factor_16k"),
        "Sp_16k": _scalar(bark, "Sp_16k"),
        "abs_thresh_power_16k": _list(loud, "abs_thresh_power_16k"),
        "zwicker_power": _scalar(loud, "zwicker_power"),
        "Sl_16k": _scalar(loud, "Sl_16k"),
        "pre_filter_b": [float(v) for v in pre.group(1).split(",")],
        "pre_filter_a": [float(v) for v in pre.group(2).split(",")],
        # loss.py:96 designs the level alignment band pass with these arguments
        "power_filter_design": {"order": 5, "band_hz": [325, 3250], "fs": 16000},
        # loss.py:291-298: windows of 20 frames, stride 10
        "psqm_window": 20,
        "psqm_stride": 10,
    }

    for key, value in tables.items():
        if isinstance(value, list) and key.endswith("16k"):
            assert len(value) == 49, (key, len(value))

    OUT.write_text(json.dumps(tables, indent=1) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
