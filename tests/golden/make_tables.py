"""Write ``tables.json``: the literal constant tables of the reference as data.

Run in the build container only (the reference tree is not present on the GPU
box); the JSON it writes is committed and is what every test loads.

Sources, parsed as text (nothing from the reference is imported or executed):

* ``torch_pesq/bark.py:11-78``   Bark band tables and ``Sp_16k``
* ``torch_pesq/loudness.py:10-25`` hearing thresholds, ``zwicker_power``, ``Sl_16k``
* ``torch_pesq/loss.py:102-108`` pre-emphasis coefficients
* ``torch_pesq/triton_ops/loss.py`` / ``reference.py:322`` loudness constant ``sl``
* ``FORMULA_SPEC`` below: every scalar constant of the loss's formulas (level
  alignment, edge ramp, chain, overlapping sums, MOS and loss), read from the
  reference's statements with ``ast`` (``loss.py``, ``loudness.py``,
  ``bark.py``, ``triton_ops/reference.py``)
"""

import ast
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


# Scalar constants of the loss's formulas, read from the reference's source
# text with ``ast`` (parsed, never executed).  Each entry selects one statement
# of one function, by the source text of its assignment target and which
# occurrence of that target it is, and names the numeric literals of that
# statement in source order; ``None`` marks a structural literal (an index,
# a ``dim=`` or ``unsqueeze`` argument, a slice bound) that is not a constant of
# the formula.  A name given twice must read the same value in both places.
FORMULA_SPEC = [
    ("torch_pesq/loss.py", "PesqLoss.align_level", "power", 0,
     [None, None, None, "align_pad", "align_divisor"]),
    ("torch_pesq/loss.py", "PesqLoss.align_level", "signal", 0,
     ["align_target_base", "align_target_exponent"]),
    ("torch_pesq/loss.py", "PesqLoss.preemphasize", "emp", 0,
     [None, "ramp_length", "ramp_points", None, "ramp_divisor"]),
    ("torch_pesq/loss.py", "PesqLoss.preemphasize", "<augassign>", 0, ["ramp_length"]),
    ("torch_pesq/loss.py", "PesqLoss.preemphasize", "<augassign>", 1, ["ramp_length", None]),
    ("torch_pesq/loss.py", "PesqLoss.raw", "deg", 0, [None, None, "pad_multiple"]),
    ("torch_pesq/loss.py", "PesqLoss.raw", "ref", 0, [None, None, "pad_multiple"]),
    ("torch_pesq/loss.py", "PesqLoss.raw", "silent", 0,
     ["silent_threshold_factor", "silent_energy"]),
    ("torch_pesq/loss.py", "PesqLoss.raw", "band_pow_ratio", 0,
     ["band_ratio_offset", "band_ratio_offset", None, "band_ratio_min", "band_ratio_max"]),
    ("torch_pesq/loss.py", "PesqLoss.raw", "frame_pow_ratio", 0,
     ["total_threshold_factor", "frame_ratio_offset", "total_threshold_factor",
      "frame_ratio_offset"]),
    ("torch_pesq/loss.py", "PesqLoss.raw", "frame_pow_ratio[:, 1:]", 0,
     [None, None, "frame_smooth_current", None, "frame_smooth_previous"]),
    ("torch_pesq/loss.py", "PesqLoss.raw", "frame_pow_ratio", 1,
     ["frame_ratio_min", "frame_ratio_max"]),
    ("torch_pesq/loss.py", "PesqLoss.raw", "deadzone", 0, ["deadzone"]),
    ("torch_pesq/loss.py", "PesqLoss.raw", "symm_distu", 0, ["symm_norm_p"]),
    ("torch_pesq/loss.py", "PesqLoss.raw", "symm_distu", 1, ["distance_floor"]),
    ("torch_pesq/loss.py", "PesqLoss.raw", "asymm_scaling", 0,
     ["asymm_offset", "asymm_offset", "asymm_exponent"]),
    ("torch_pesq/loss.py", "PesqLoss.raw", "asymm_scaling[asymm_scaling < 3.0]", 0,
     ["asymm_cut", "asymm_cut_value"]),
    ("torch_pesq/loss.py", "PesqLoss.raw", "asymm_scaling", 1, ["asymm_cap"]),
    ("torch_pesq/loss.py", "PesqLoss.raw", "asymm_distu", 0, ["asymm_norm_p"]),
    ("torch_pesq/loss.py", "PesqLoss.raw", "asymm_distu", 1, ["distance_floor"]),
    ("torch_pesq/loss.py", "PesqLoss.raw", "h", 0,
     ["total_threshold_factor", "h_offset", "h_scale", "h_exponent"]),
    ("torch_pesq/loss.py", "PesqLoss.raw", "(symm_distu, asymm_distu)", 0,
     ["distance_cap", "distance_cap"]),
    ("torch_pesq/loss.py", "PesqLoss.raw", "psqm", 0,
     [None, None, None, "psqm_window", "psqm_stride", "psqm_power", None, None, "psqm_power"]),
    ("torch_pesq/loss.py", "PesqLoss.raw", "psqm", 1,
     [None, None, None, "psqm_window", "psqm_stride", "psqm_power", None, None, "psqm_power"]),
    ("torch_pesq/loss.py", "PesqLoss.mos", "mos", 0,
     ["pesq_offset", "pesq_symm_weight", "pesq_asymm_weight"]),
    ("torch_pesq/loss.py", "PesqLoss.mos", "mos", 1,
     ["mos_floor", "mos_span", None, "mos_slope", "mos_shift"]),
    ("torch_pesq/loss.py", "PesqLoss.forward", "<return>", 0,
     ["pesq_symm_weight", "pesq_asymm_weight"]),
    ("torch_pesq/loudness.py", "Loudness.__init__", "exp", 0,
     ["exponent_numerator", "exponent_offset"]),
    ("torch_pesq/loudness.py", "Loudness.__init__", "self.exp", 0,
     ["exponent_min", "exponent_max", "exponent_power"]),
    ("torch_pesq/loudness.py", "Loudness.time_avg_audible", "mask", 0,
     ["mean_threshold_factor"]),
    ("torch_pesq/loudness.py", "Loudness.forward", "loudness", 0,
     ["loudness_threshold_scale", "loudness_half", "loudness_half", "loudness_one"]),
    ("torch_pesq/loudness.py", "Loudness.forward", "loudness[pow_dens <= self.threshs]", 0,
     ["loudness_below_threshold"]),
    ("torch_pesq/bark.py", "BarkScale.weighted_norm", "<return>", 0,
     [None, "norm_first_band", None]),
    # the Triton backend's float64 reference restates the chain; it must agree
    ("torch_pesq/triton_ops/reference.py", "ref_chain", "silent", 0,
     ["silent_threshold_factor", "silent_energy"]),
    ("torch_pesq/triton_ops/reference.py", "ref_chain", "mask_ref", 0,
     ["mean_threshold_factor", None]),
    ("torch_pesq/triton_ops/reference.py", "ref_chain", "band_pow_ratio", 0,
     ["band_ratio_offset", "band_ratio_offset", None, "band_ratio_min", "band_ratio_max"]),
    ("torch_pesq/triton_ops/reference.py", "ref_chain", "frame_pow_ratio", 1,
     [None, None, "frame_smooth_current", None, "frame_smooth_previous", None,
      "frame_ratio_min", "frame_ratio_max"]),
    ("torch_pesq/triton_ops/reference.py", "ref_chain", "deadzone", 0, ["deadzone"]),
    ("torch_pesq/triton_ops/reference.py", "ref_chain", "asymm_scaling", 0,
     ["asymm_offset", "asymm_offset", "asymm_exponent"]),
    ("torch_pesq/triton_ops/reference.py", "ref_chain", "asymm_scaling", 1,
     ["asymm_cut", "asymm_cap"]),
    ("torch_pesq/triton_ops/reference.py", "ref_chain", "h", 0,
     ["h_offset", "h_scale", "h_exponent"]),
    ("torch_pesq/triton_ops/reference.py", "_loudness", "loudness", 0,
     ["loudness_threshold_scale", "loudness_half", "loudness_half", "loudness_one"]),
    ("torch_pesq/triton_ops/reference.py", "ref_pipeline", "<return>", 0, ["sl"]),
]


def _function(tree, qualname):
    node = tree
    for part in qualname.split("."):
        for child in ast.iter_child_nodes(node):
            if isinstance(child, (ast.FunctionDef, ast.ClassDef)) and child.name == part:
                node = child
                break
        else:
            raise SystemExit(f"{qualname} not found")
    return node


def _target(statement):
    if isinstance(statement, ast.Assign):
        return ast.unparse(statement.targets[0])
    if isinstance(statement, ast.AugAssign):
        return "<augassign>"
    if isinstance(statement, ast.Return):
        return "<return>"
    return None


def _literals(statement):
    found = [
        (n.lineno, n.col_offset, n.value)
        for n in ast.walk(statement)
        if isinstance(n, ast.Constant)
        and isinstance(n.value, (int, float))
        and not isinstance(n.value, bool)
    ]
    return [(line, value) for line, _, value in sorted(found)]


def formula_constants(ref_root):
    """``{name: value}`` and ``{name: "file:line, ..."}`` of ``FORMULA_SPEC``."""

    trees, values, sources = {}, {}, {}
    for path, qualname, target, occurrence, names in FORMULA_SPEC:
        if path not in trees:
            trees[path] = ast.parse((ref_root / path).read_text())
        body = _function(trees[path], qualname).body
        matches = [st for st in body if _target(st) == target]
        if occurrence >= len(matches):
            raise SystemExit(f"{path} {qualname}: no statement #{occurrence} assigning {target}")
        statement = matches[occurrence]
        literals = _literals(statement)
        if len(literals) != len(names):
            raise SystemExit(f"{path}:{statement.lineno}: literals {literals} vs names {names}")
        for name, (line, value) in zip(names, literals):
            if name is None:
                continue
            if name in values and values[name] != value:
                raise SystemExit(f"{name}: {values[name]} and {value} ({path}:{line})")
            values[name] = value
            where = f"{path}:{line}"
            if where not in sources.get(name, "").split(", "):
                sources[name] = where if name not in sources else f"{sources[name]}, {where}"
    return values, sources


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
    tables["formula_constants"], tables["formula_constant_sources"] = formula_constants(REF)

    for key, value in tables.items():
        if isinstance(value, list) and key.endswith("16k"):
            assert len(value) == 49, (key, len(value))

    OUT.write_text(json.dumps(tables, indent=1) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
