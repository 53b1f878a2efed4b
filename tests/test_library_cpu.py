"""CPU checks of the C ABI library and of the host side of the package.

No kernel is launched here: the library must load, export every entry point
``include/pesq_hip.h`` declares, pack its constant tables, and reject invalid
arguments before touching a GPU.
"""

import ctypes
import json
import re
from pathlib import Path

import numpy as np
import pytest
import torch
from scipy.signal import butter, lfilter, sosfilt

from torch_pesq import BarkScale, Loudness, PesqLoss, _lib
from torch_pesq import bark as bark_mod
from torch_pesq import loudness as loud_mod
from torch_pesq.hip_ops.iir import HipIIR, parallel_sections, realise

ROOT = Path(__file__).resolve().parents[1]
TABLES = json.loads((ROOT / "tests" / "golden" / "tables.json").read_text())


def _declared_symbols():
    header = (ROOT / "include" / "pesq_hip.h").read_text()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(pesq_\w+)\s*\(", header, re.M)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.library()
    declared = _declared_symbols()
    assert len(declared) >= 15
    for name in declared:
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert lib.pesq_abi_version() >= 1


def test_torch_extension_loads_and_shares_the_library():
    ext = _lib.torch_ext()
    assert callable(ext.pipeline)
    # the extension resolves libpesq_hip.so by soname to the copy ctypes loaded
    maps = Path("/proc/self/maps").read_text().splitlines()
    paths = {line.split()[-1] for line in maps if line.endswith("libpesq_hip.so")}
    assert paths == {str(_lib.LIB_PATH.resolve())}
    # host tensors are refused before any library call
    table = torch.zeros(_lib.library().pesq_model_table_bytes(), dtype=torch.uint8)
    x = torch.zeros(1, 16000, requires_grad=True)
    with pytest.raises(RuntimeError, match="must be GPU tensors"):
        ext.pipeline(x, x.detach(), table, 1.0)

    from torch_pesq.hip_ops.resample import HipResample

    rs = HipResample(48000, 16000)
    assert rs.plan_bytes.numel() == ctypes.sizeof(_lib.ResamplePlanInfo)
    assert not rs.plan_bytes.is_cuda
    tables = (rs.kernel, rs.tap_lo, rs.tap_hi, rs.phase_lo, rs.phase_hi, rs.plan, rs.plan_bytes)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        ext.resample(torch.zeros(2, 4800), 1600, *tables, rs.orig_step, rs.new_step, rs.width)


def test_product_tables_match_golden():
    for key in (
        "nr_of_hz_bands_per_bark_band_16k",
        "centre_of_band_bark_16k",
        "centre_of_band_hz_16k",
        "width_of_band_bark_16k",
        "width_of_band_hz_16k",
        "pow_dens_correction_factor_16k",
    ):
        assert list(getattr(bark_mod, key)) == TABLES[key], key
    assert bark_mod.Sp_16k == TABLES["Sp_16k"]
    assert list(loud_mod.abs_thresh_power_16k) == TABLES["abs_thresh_power_16k"]
    assert loud_mod.zwicker_power == TABLES["zwicker_power"]
    assert loud_mod.Sl_16k == TABLES["Sl_16k"]


def test_fbank_known_answer():
    # tests/test_fbank.py:5-11 of the reference
    fb = BarkScale()
    assert torch.all(fb.fbank.sum(dim=1) == torch.tensor(bark_mod.nr_of_hz_bands_per_bark_band_16k))
    assert torch.all(fb.fbank.sum(dim=0) == 1.0)
    assert fb.pow_dens_correction.dtype == torch.float64
    assert Loudness().exp.dtype == torch.float32


def test_model_matches_oracle_constants():
    from oracle import pesq_oracle as O

    c = O.constants()
    m = PesqLoss(1.0, sample_rate=16000)
    assert torch.equal(m.power_filter.double(), torch.stack([c["power_b"], c["power_a"]]))
    assert torch.equal(m.pre_filter.double(), torch.stack([c["pre_b"], c["pre_a"]]))
    assert torch.equal(m.to_spec.window.double(), c["window"])
    assert torch.equal(m.fbank.fbank.double(), c["fbank"])
    assert torch.equal(m.fbank.pow_dens_correction, c["corr"])
    assert torch.equal(m.loudness.threshs.flatten(), c["threshs"])
    assert torch.equal(m.loudness.exp.double(), c["exp"])
    assert float(m.fbank.total_width) == float(c["total_width"])


@pytest.mark.parametrize(
    "b,a",
    [
        butter(5, [325, 3250], fs=16000, btype="band"),
        ([2.740826, -5.4816519, 2.740826], [1.0, -1.9444777, 0.94597794]),
        butter(4, 0.2),
        butter(3, [0.1, 0.4], btype="bandstop"),
        ([0.5, 0.1], [1.0, -0.9]),
        butter(8, 0.3),
    ],
)
def test_parallel_realisation_reproduces_lfilter(b, a):
    c0, secs = parallel_sections(b, a)
    x = np.random.default_rng(0).standard_normal(5000)
    want = lfilter(b, a, x)
    got = c0 * x + sum(lfilter([s[0], s[1], s[2]], [1.0, s[3], s[4]], x) for s in secs)
    assert np.abs(got - want).max() <= 1e-9 * np.abs(want).max()
    assert len(secs) == (len(np.trim_zeros(np.asarray(a, float), "b")) - 1 + 1) // 2


def test_parallel_realisation_rejects_repeated_poles():
    # (1 - 0.5 z^-1)^-3: a triple real pole has no parallel first/second order form
    a = np.poly([0.5, 0.5, 0.5])
    with pytest.raises(RuntimeError):
        parallel_sections([1.0], a)


@pytest.mark.parametrize(
    "b,a,basis",
    [
        (*butter(5, [325, 3250], fs=16000, btype="band"), "parallel"),
        (*butter(8, [325, 3250], fs=16000, btype="band"), "cascade"),
        ([1.0, 0.0, 0.0, 0.0], np.poly([0.7, 0.7, 0.7]), "cascade"),
        ([1.0, 2.0, 3.0, 4.0, 5.0], [1.0, -0.5, 0.0, 0.0, 0.0], "cascade"),
        ([1.0, 2.0, 3.0], [1.0, -0.5, 0.0], "cascade"),
        ([2.740826, -5.4816519, 2.740826], [1.0, -1.9444777, 0.94597794], "cascade"),
    ],
)
def test_realisation_choice_and_fidelity(b, a, basis):
    """The chosen realisation reproduces the float64 difference equation.

    The parallel form needs distinct poles and no FIR tail; repeated poles
    (the triple pole), numerators longer than the denominator and order 16
    band passes (clustered poles) take the cascade, order <= 2 a single full
    biquad.  The check runs the realisation itself (sums of biquads, or
    ``sosfilt`` over the sections) on noise against ``lfilter`` of (b, a).
    """

    real = realise(b, a)
    assert real.basis == basis
    x = np.random.default_rng(3).standard_normal(6000)
    want = lfilter(np.asarray(b, float), np.asarray(a, float), x)
    if real.basis == "parallel":
        got = real.c0 * x + sum(lfilter(s[:3], [1.0, s[3], s[4]], x) for s in real.sections)
    else:
        got = sosfilt(real.sections, x)
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err <= max(10 * real.score, 1e-12), (err, real.score)
    assert real.score < 1e-6


def test_realisation_rating_matches_the_reference_limits():
    """Order 20 band pass: usable but degraded (warns); order 30: rejected.

    The reference's ``test_degraded_filter_warns`` and
    ``test_unrepresentable_filter_raises_instead_of_returning_nan``
    (``test_triton_iir.py:860-884``) with its limits 1e3 and 1e5 times 2^-24.
    """

    with pytest.warns(RuntimeWarning, match="degraded"):
        HipIIR(*butter(10, [325, 3250], fs=16000, btype="band"))
    with pytest.raises(RuntimeError, match="realisation"):
        HipIIR(*butter(15, [325, 3250], fs=16000, btype="band"))


def test_realisation_argument_errors():
    with pytest.raises(ValueError):
        realise([1.0, 0.5], [0.0, 1.0])
    with pytest.raises(ValueError):
        realise([1.0], [1.0])
    with pytest.raises(ValueError):
        HipIIR([1.0, 0.5], [1.0, -0.5], chunk_size=100)
    with pytest.raises(ValueError):
        HipIIR([1.0, 0.5], [1.0, -0.5], method="direct")
    mod = HipIIR(*butter(8, [325, 3250], fs=16000, btype="band"), chunk_size="tune")
    assert (mod.order, mod.states, mod.sections) == (16, 16, 8)
    assert mod.candidates == (64, 128, 256, 512)


def test_iir_cascade_pack_validates():
    lib = _lib.library()
    size = lib.pesq_iir_table_bytes()
    sos = np.array([[1.0, 0.5, 0.25, 1.0, -0.5, 0.1]] * 2)
    buf = (ctypes.c_ubyte * (2 * size))()
    ptr = sos.ctypes.data_as(ctypes.c_void_p)
    assert lib.pesq_iir_cascade_pack(ptr, 2, buf) == 0
    assert lib.pesq_iir_cascade_pack(ptr, 0, buf) != 0
    assert b"sections" in lib.pesq_last_error()
    assert lib.pesq_iir_cascade_pack(ptr, _lib.MAX_CASCADE + 1, buf) != 0
    bad = sos.copy()
    bad[1, 3] = 0.0
    assert lib.pesq_iir_cascade_pack(bad.ctypes.data_as(ctypes.c_void_p), 2, buf) != 0
    assert b"leading denominator" in lib.pesq_last_error()
    out = ctypes.c_size_t(0)
    assert lib.pesq_iir_cascade_workspace(4, 5000, 3, ctypes.byref(out)) == 0
    # the scan workspace of one section plus two float64 intermediate signals
    nblk = -(-5000 // 1024)
    assert out.value == (4 * nblk * 2 * 65 + 2 * 4 * 5000) * 8
    assert lib.pesq_iir_cascade_workspace(4, 5000, 0, ctypes.byref(out)) != 0


def test_stft_construction_validation():
    """The constructor checks of ``test_triton_spectral.py:200-260``, same messages."""

    from torch_pesq.hip_ops.spectral import HipStftBark

    window = torch.hann_window(64)
    corr = torch.ones(4)
    overlapping = torch.zeros(4, 32)
    overlapping[0, 0:8] = 1.0
    overlapping[1, 4:12] = 1.0
    with pytest.raises(ValueError, match="disjoint"):
        HipStftBark(window, overlapping, corr, 64, 32)
    gappy = torch.zeros(4, 32)
    gappy[0, 0] = gappy[0, 5] = 1.0
    with pytest.raises(ValueError, match="not contiguous"):
        HipStftBark(window, gappy, corr, 64, 32)
    weighted = torch.zeros(4, 32)
    weighted[0, 0:4] = 0.5
    with pytest.raises(ValueError, match="binary"):
        HipStftBark(window, weighted, corr, 64, 32)
    fine = torch.zeros(4, 32)
    fine[0, 0:4] = 1.0
    with pytest.raises(ValueError, match="at least 32"):
        HipStftBark(window[:16], fine[:, :8], corr, 16, 8)
    with pytest.raises(ValueError, match="512 bins"):
        HipStftBark(window, fine, corr, 1024, 32)
    with pytest.raises(ValueError, match="one entry per band"):
        HipStftBark(window, fine, corr[:2], 64, 32)
    with pytest.raises(ValueError, match="at most 64 taps"):
        HipStftBark(torch.hann_window(128), fine, corr, 64, 32)
    for n_fft in (40, 48, 96, 1000):
        fb = torch.zeros(4, n_fft // 2)
        for band in range(4):
            fb[band, 4 * band : 4 * band + 4] = 1.0
        with pytest.raises(ValueError, match="power of two"):
            HipStftBark(torch.hann_window(n_fft), fb, torch.ones(4), n_fft, n_fft // 2)
    # accepted: the general kernels for anything but the PESQ geometry
    mod = HipStftBark(window, fine, corr, 64, 32)
    assert mod.general and mod.novertaps == 2
    scale = BarkScale(256, 49)
    assert not HipStftBark(torch.hann_window(512), scale.fbank, scale.pow_dens_correction).general


def test_chain_table_pack_validates():
    lib = _lib.library()
    buf = (ctypes.c_ubyte * lib.pesq_model_table_bytes())()
    th = np.full(17, 2.0)
    ex = np.full(17, 0.2)
    wd = np.full(17, 0.5)
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    assert lib.pesq_chain_table_pack(17, ptr(th), ptr(ex), ptr(wd), 8.0, 0.18, buf) == 0
    assert lib.pesq_chain_table_pack(128, ptr(np.ones(128)), ptr(np.ones(128)), ptr(np.ones(128)),
                                     8.0, 0.18, buf) == 0
    assert lib.pesq_chain_table_pack(129, ptr(np.ones(129)), ptr(np.ones(129)), ptr(np.ones(129)),
                                     8.0, 0.18, buf) != 0
    assert b"bands" in lib.pesq_last_error()
    th[3] = 0.0
    assert lib.pesq_chain_table_pack(17, ptr(th), ptr(ex), ptr(wd), 8.0, 0.18, buf) != 0
    assert b"strictly positive" in lib.pesq_last_error()
    out = ctypes.c_size_t(0)
    assert lib.pesq_chain_forward_workspace(2, 40, 17, ctypes.byref(out)) == 0
    assert lib.pesq_chain_forward_workspace(2, 40, 0, ctypes.byref(out)) != 0


def test_iir_table_pack_validates():
    lib = _lib.library()
    s = _lib.IirSections()
    s.count = 0
    buf = (ctypes.c_ubyte * lib.pesq_iir_table_bytes())()
    assert lib.pesq_iir_table_pack(ctypes.byref(s), buf) != 0
    assert b"sections" in lib.pesq_last_error()
    s.count = 1
    s.b0[0], s.a1[0], s.a2[0] = 1.0, -0.5, 0.0
    assert lib.pesq_iir_table_pack(ctypes.byref(s), buf) == 0


def test_pipeline_workspace_queries_validate():
    lib = _lib.library()
    size = ctypes.c_size_t(0)
    assert lib.pesq_pipeline_forward_workspace(8, 128000, 2, ctypes.byref(size)) == 0
    assert size.value > 8 * 128000 * 2 * 4
    # fewer than 20 frames
    assert lib.pesq_pipeline_forward_workspace(1, 4000, 0, ctypes.byref(size)) != 0
    assert b"20 frames" in lib.pesq_last_error()
    # an empty batch is valid (its calls are no-ops), a negative one is not
    assert lib.pesq_pipeline_forward_workspace(0, 16000, 0, ctypes.byref(size)) == 0
    assert lib.pesq_pipeline_forward_workspace(-1, 16000, 0, ctypes.byref(size)) != 0
    assert b"negative" in lib.pesq_last_error()
    # the empty batch returns before any pointer is read: NULLs are fine
    assert lib.pesq_pipeline_forward(None, None, 0, 16000, None, 1.0, 2, None, None, None, None,
                                     None, None) == 0
    assert lib.pesq_pipeline_backward(None, None, None, None, 0, 16000, None, 1.0, 2, None, None,
                                      None, None, None) == 0
    assert lib.pesq_chain_forward(None, None, 0, 62, 49, ctypes.c_void_p(1), None, None, None,
                                  None) == 0
    off, nbytes = ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert lib.pesq_pipeline_region(2, 16000, 2, b"bark", ctypes.byref(off), ctypes.byref(nbytes)) == 0
    assert nbytes.value >= 4 * 62 * 49 * 4
    assert lib.pesq_pipeline_region(2, 16000, 2, b"nope", ctypes.byref(off), ctypes.byref(nbytes)) != 0


def test_model_table_pack_rejects_bad_bands():
    from torch_pesq.hip_ops.pipeline import pack_model_table

    m = PesqLoss(1.0, sample_rate=16000)
    fb = m.fbank.fbank.clone()
    fb[3, 0] = 1.0  # band 3 reaches back into band 0's bin
    with pytest.raises(ValueError):
        pack_model_table(m.power_filter[0], m.power_filter[1], m.pre_filter[0], m.pre_filter[1],
                         m.to_spec.window, fb, m.fbank.pow_dens_correction, m.loudness.threshs,
                         m.loudness.exp, m.fbank.width_bark, m.fbank.total_width, 0.1866055)


def _pair_decay(poles, n=2048):
    """Largest entry of A^n for the 2x2 companion block of each pole pair
    (z^2 + a1 z + a2 with the pair's roots), over the pairs."""

    poles = sorted(poles, key=lambda p: (abs(p.imag), p.real))
    worst = 0.0
    for i in range(0, len(poles), 2):
        a1 = -(poles[i] + poles[i + 1]).real
        a2 = (poles[i] * poles[i + 1]).real
        comp = np.array([[-a1, 1.0], [-a2, 0.0]])
        worst = max(worst, np.abs(np.linalg.matrix_power(comp, n)).max())
    return worst


def _pack(m, power_a=None, pre_a=None):
    from torch_pesq.hip_ops.pipeline import pack_model_table

    return pack_model_table(
        m.power_filter[0], m.power_filter[1] if power_a is None else power_a,
        m.pre_filter[0], m.pre_filter[1] if pre_a is None else pre_a,
        m.to_spec.window, m.fbank.fbank, m.fbank.pow_dens_correction, m.loudness.threshs,
        m.loudness.exp, m.fbank.width_bark, m.fbank.total_width, 0.1866055)


def test_filters_decay_within_the_window():
    """The scans start each block from the two blocks before it run from a
    zero state (and the backward's output pass starts the pre-emphasis
    filter 2048 samples early): every section's state must keep at most 1e-20
    of itself over 2048 samples, which the pack checks.  The standard filters
    keep at most 3e-24 (largest entry of A^2048 over the pole pairs; pole
    radii 0.968 for the level alignment filter, 0.973 for the pre-emphasis
    filter), and filters decaying more slowly are refused where the table is
    packed."""

    m = PesqLoss(1.0, sample_rate=16000)
    pre_poles = np.roots(m.pre_filter[1].double().numpy())
    power_poles = np.roots(m.power_filter[1].double().numpy())
    assert abs(np.abs(pre_poles).max() - 0.9726) < 1e-3
    assert abs(np.abs(power_poles).max() - 0.968) < 2e-3
    assert _pair_decay(pre_poles) < 3e-24
    assert _pair_decay(power_poles) < 3e-24
    _pack(m)

    slow_pre = torch.tensor([1.0, -1.98 * np.cos(0.1), 0.99 ** 2], dtype=torch.float64)
    assert _pair_decay(np.roots(slow_pre.numpy())) > 1e-20
    with pytest.raises((RuntimeError, ValueError), match="pre-emphasis filter decays too slowly"):
        _pack(m, pre_a=slow_pre)
    # a level alignment filter of the same order with well separated poles
    # at radius 0.995
    angles = np.array([0.3, 0.9, 1.5, 2.1, 2.7])
    slow_poles = 0.995 * np.exp(1j * np.concatenate([angles, -angles]))
    slow_power = torch.from_numpy(np.poly(slow_poles).real.copy())
    assert _pair_decay(slow_poles) > 1e-20
    with pytest.raises((RuntimeError, ValueError),
                       match="level alignment filter decays too slowly"):
        _pack(m, power_a=slow_power)


def test_cpu_inputs_and_bad_shapes_raise():
    m = PesqLoss(1.0, sample_rate=16000)
    ref = torch.zeros(2, 16000)
    with pytest.raises(RuntimeError):
        m(ref, ref)
    with pytest.raises(ValueError):
        m(ref, torch.zeros(2, 15000))
    # the loudness exponents keep the standard's 49 bands, so other band
    # counts are refused by the chain, as in the reference
    with pytest.raises(ValueError, match="same number of bands"):
        PesqLoss(1.0, nbarks=32)
    # other STFT geometries are accepted (general kernels)
    assert PesqLoss(1.0, sample_rate=16000, n_fft=256, win_length=200, hop_length=128).general


def test_graft_entry_exposes_build_and_smoke():
    import __graft_entry__ as entry

    assert callable(entry.build) and callable(entry.smoke)


# -- kernel variants per shape (host query, no GPU call) ----------------------

#: (batch, 16 kHz length, grad mask) -> kernels of the forward and the backward
#: pass.  The variants are chosen by grid size: lane states are stored for
#: grids of up to 8192 scan wavefronts and recomputed above; grids that store
#: them take windowed block starts in the output pass (the output kernel's
#: fifth argument 2, kWindowStarts: the two previous blocks' aggregates), the
#: others a prefix kernel (0, kStoredStarts); the STFT and chain kernels of
#: grids above 512 chain tiles take four frames per wavefront (the STFT
#: backward two).  Where the backward scan stores lane states and has rows of
#: up to 128 blocks (c2, c3), the forward's STFT kernel also runs the
#: backward's level alignment aggregate and the backward's output pass warms
#: the pre-emphasis filter up itself, so the backward has no aggregate launch
#: (iir_output_split_kernel: the two filters on two wavefronts per block).
#: The aggregate pass of lane-state grids runs three wavefronts per block,
#: each on its own sections (iir_aggregate_split_kernel).
VARIANTS = {
    # BASELINE c2: 16 rows x 125 blocks, 8 x 32 tiles
    (8, 128000, 2): (
        ["iir_aggregate_split_kernel<5, 1, 3, PipeFwdMode>",
         "iir_output_kernel<5, 1, PipeFwdMode, true, 2, false>",
         "stft_fwd_kernel<float, false, 8>", "chain_fwd_kernel<8, 1>", "chain_final_kernel"],
        ["chain_bwd_kernel<16, 1>", "stft_bwd_kernel<float, 1, 9>",
         "iir_output_split_kernel<5, 1, PipeBwdMode, true>"],
    ),
    # BASELINE c4: 938 blocks per row, 4 x 235 = 940 tiles, items
    # of 235 tiles (per item band totals)
    (4, 960000, 2): (
        ["iir_aggregate_split_kernel<5, 1, 3, PipeFwdMode>",
         "iir_output_kernel<5, 1, PipeFwdMode, true, 2, false>",
         "stft_fwd_kernel<float, true, 8>", "band_totals_kernel<16, 2>",
         "chain_fwd_kernel<4, 1>", "chain_final_kernel"],
        ["chain_bwd_kernel<4, 1>", "band_totals_kernel<8, 1>", "stft_bwd_kernel<float, 2, 8>",
         "iir_aggregate_split_kernel<5, 1, 3, PipeBwdMode>",
         "iir_output_kernel<5, 1, PipeBwdMode, true, 2, false>"],
    ),
    # one item of 65 tiles (1033 frames): just past the band totals threshold
    (1, 264704, 1): (
        ["iir_aggregate_split_kernel<5, 1, 3, PipeFwdMode>",
         "iir_output_kernel<5, 1, PipeFwdMode, true, 2, false>",
         "stft_fwd_kernel<float, false, 8>", "band_totals_kernel<16, 2>",
         "chain_fwd_kernel<8, 1>", "chain_final_kernel"],
        ["chain_bwd_kernel<16, 1>", "band_totals_kernel<8, 1>", "stft_bwd_kernel<float, 1, 9>",
         "iir_aggregate_split_kernel<5, 1, 3, PipeBwdMode>",
         "iir_output_kernel<5, 1, PipeBwdMode, true, 2, false>"],
    ),
    # one item of 64 tiles (1023 frames): the largest without band totals
    (1, 262144, 1): (
        ["iir_aggregate_split_kernel<5, 1, 3, PipeFwdMode>",
         "iir_output_kernel<5, 1, PipeFwdMode, true, 2, false>",
         "stft_fwd_kernel<float, false, 8>", "chain_fwd_kernel<8, 1>", "chain_final_kernel"],
        ["chain_bwd_kernel<16, 1>", "stft_bwd_kernel<float, 1, 9>",
         "iir_aggregate_split_kernel<5, 1, 3, PipeBwdMode>",
         "iir_output_kernel<5, 1, PipeBwdMode, true, 2, false>"],
    ),
    # BASELINE c5 after the 3:1 resampler: 512 x 63 = 32256 forward scan
    # wavefronts, 256 x 63 = 16128 backward ones (both above 8192)
    (256, 64000, 2): (
        ["iir_aggregate_kernel<5, 1, PipeFwdMode, false, 0, 6>", "iir_prefix_kernel<6>",
         "iir_output_kernel<5, 1, PipeFwdMode, false, 0, false>",
         "stft_fwd_kernel<float, true, 8>", "chain_fwd_kernel<4, 1>", "chain_final_kernel"],
        ["chain_bwd_kernel<4, 1>", "stft_bwd_kernel<float, 2, 8>",
         "iir_aggregate_kernel<5, 1, PipeBwdMode, false, 0, 6>", "iir_prefix_kernel<6>",
         "iir_output_kernel<5, 1, PipeBwdMode, false, 0, false>"],
    ),
    # BASELINE c3 after the 441:160 resampler: a small grid like c2
    (16, 64000, 2): (
        ["iir_aggregate_split_kernel<5, 1, 3, PipeFwdMode>",
         "iir_output_kernel<5, 1, PipeFwdMode, true, 2, false>",
         "stft_fwd_kernel<float, false, 8>", "chain_fwd_kernel<8, 1>", "chain_final_kernel"],
        ["chain_bwd_kernel<16, 1>", "stft_bwd_kernel<float, 1, 9>",
         "iir_output_split_kernel<5, 1, PipeBwdMode, true>"],
    ),
}


@pytest.mark.parametrize("shape", sorted(VARIANTS))
def test_pipeline_kernel_variants_per_shape(shape):
    fwd, bwd = VARIANTS[shape]
    assert _lib.pipeline_kernels(*shape, backward=False) == fwd
    assert _lib.pipeline_kernels(*shape, backward=True) == bwd


def test_pipeline_kernel_query_edges():
    lib = _lib.library()
    needed = ctypes.c_size_t(0)
    assert lib.pesq_pipeline_kernels(8, 128000, 2, 0, None, 0, ctypes.byref(needed)) == 0
    full = ctypes.create_string_buffer(int(needed.value))
    assert lib.pesq_pipeline_kernels(8, 128000, 2, 0, full, len(full), None) == 0
    assert len(full.value) + 1 == needed.value
    # a short buffer gets a truncated, terminated prefix
    short = ctypes.create_string_buffer(10)
    assert lib.pesq_pipeline_kernels(8, 128000, 2, 0, short, len(short), None) == 0
    assert short.value == full.value[:9]
    # the backward needs a gradient; too few frames are rejected like the pipeline does
    assert lib.pesq_pipeline_kernels(8, 128000, 0, 1, None, 0, None) == _lib.ERR_ARGUMENT
    assert lib.pesq_pipeline_kernels(1, 4000, 2, 0, None, 0, None) == _lib.ERR_ARGUMENT
    # 4 bands more than a lane's worth is not a pipeline shape: the pipeline is 49 bands
    names = _lib.pipeline_kernels(1, 16000, 1, backward=True)
    assert names[0] == "chain_bwd_kernel<16, 1>"


def test_lane_state_region_only_when_stored():
    """The scan workspace holds 64 lane states per block only for grids that store them."""

    def fwd_bytes(batch, length):
        return _lib.size_query(_lib.library().pesq_pipeline_forward_workspace, batch, length, 2)

    # 16 rows x 125 blocks x 6 sections x 2 doubles x (1 aggregate + 64 lane states)
    assert _region_size(8, 128000, "aggr") == 16 * 125 * 6 * 2 * 65 * 8
    # c5: 512 rows x 63 blocks, recomputed lane states: aggregates only
    assert _region_size(256, 64000, "aggr") == 512 * 63 * 6 * 2 * 8
    assert fwd_bytes(256, 64000) < 600 * 2**20


def _region_size(batch, length, name):
    off = ctypes.c_size_t(0)
    size = ctypes.c_size_t(0)
    _lib.check(_lib.library().pesq_pipeline_region(batch, length, 2, name.encode(),
                                                    ctypes.byref(off), ctypes.byref(size)))
    return size.value


def test_triton_ops_import_paths_resolve_to_the_hip_operators():
    """The reference's operator modules import unchanged (``torch_pesq.triton_ops.*``)."""

    from torch_pesq import triton_ops
    from torch_pesq.hip_ops import chain, elementwise, iir, resample, spectral
    from torch_pesq.hip_ops.loss import PesqLossHip
    from torch_pesq.triton_ops import _common as t_common
    from torch_pesq.triton_ops import chain as t_chain
    from torch_pesq.triton_ops import elementwise as t_elem
    from torch_pesq.triton_ops import iir as t_iir
    from torch_pesq.triton_ops import loss as t_loss
    from torch_pesq.triton_ops import resample as t_resample
    from torch_pesq.triton_ops import spectral as t_spectral

    assert triton_ops.HAS_TRITON == torch.cuda.is_available()
    assert t_iir.TritonIIR is iir.HipIIR
    assert t_iir.CHUNK_CANDIDATES == (64, 128, 256, 512) and t_iir.METHODS == ("scan", "matmul")
    assert t_resample.TritonResample is resample.HipResample
    assert t_spectral.TritonStftBark is spectral.HipStftBark
    assert t_spectral.bark_segments is spectral.bark_segments
    assert t_chain.TritonPesqChain is chain.HipPesqChain
    for name in ("peak_normalize", "edge_ramp", "align_scale", "pesq_epilogue"):
        assert getattr(t_elem, name) is getattr(elementwise, name)
    assert t_loss.PesqLossTriton is PesqLossHip
    from torch_pesq import PesqLossTriton

    assert PesqLossTriton is PesqLossHip
    assert callable(t_common.check_input) and callable(t_common.require_triton)
    # constructors take the reference's arguments and need no GPU
    t_iir.TritonIIR([0.2, 0.3], [1.0, -0.5])
    t_resample.TritonResample(44100, 16000)
    with pytest.raises(RuntimeError, match="GPU"):
        t_common.check_input(torch.zeros(3))


def test_kernel_trace_normalises_library_names():
    """The profiler's kernel names and the library's list compare in one spelling."""

    from kernel_trace import library_kernels, normalise

    assert normalise("void pesq::iir_prefix_kernel<6>(pesq::IirTable const*, double*, int, long)") \
        == "iir_prefix_kernel<6>"
    mangled = "_ZN4pesq20iir_aggregate_kernelILi5ELi1ENS_11PipeFwdModeELb1ELi0ELi6EEEvT1_PKNS_8IirTableEPdS6_li"
    assert normalise(mangled) == "iir_aggregate_kernel<5,1,PipeFwdMode,true,0,6>"
    assert library_kernels(8, 128000, 2, False)[0] == "iir_aggregate_split_kernel<5,1,3,PipeFwdMode>"
    assert all(" " not in k for k in library_kernels(4, 960000, 2, True))


@pytest.mark.parametrize("orig,new", [(44100, 16000), (22050, 16000), (8000, 16000), (13, 7), (7, 13)])
def test_resample_plan_transposed_bank_is_the_adjoint(orig, new):
    """The plan's adjoint bank (host packing, no GPU): applying it as a resampler
    from the new rate to the old one, ``gx[l o + j] = sum_t adj[t][j]
    gy[l n + adj_offs[j] + t]``, gives the float64 adjoint of the oracle's
    resampler on a random upstream gradient."""

    from oracle import pesq_oracle as O
    from torch_pesq.hip_ops.resample import HipResample

    mod = HipResample(orig, new)
    info = mod.plan_info
    o, n = info.orig_step, info.new_step
    assert info.adj_span > 0 and info.adj_taps >= 1
    plan = mod.plan.numpy()
    adj = plan[info.off_adj_taps:info.off_adj_taps + 4 * info.adj_taps * o].view(np.float32)
    adj = adj.reshape(info.adj_taps, o).astype(np.float64)
    offs = plan[info.off_adj_offs:info.off_adj_offs + 4 * o].view(np.int32)
    length = 2 * 441 + 17
    x = torch.randn(1, length, dtype=torch.float64, requires_grad=True)
    y = O.resample(x, orig, new)
    gy = torch.randn(y.shape, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    (want,) = torch.autograd.grad(y, x, grad_outputs=gy)
    g = gy[0].numpy()
    got = np.zeros(length)
    for i in range(length):
        l, j = divmod(i, o)
        m = l * n + offs[j] + np.arange(info.adj_taps)
        ok = (m >= 0) & (m < g.shape[0])
        got[i] = np.dot(adj[:, j][ok], g[m[ok]])
    # the oracle's bank is the float32 bank promoted: the same products
    np.testing.assert_allclose(got, want[0].numpy(), rtol=0, atol=1e-12 * np.abs(g).max())
