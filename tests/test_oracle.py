"""Pins of the float64 CPU oracle (``oracle/pesq_oracle.py``).

Each check is chosen so that a plausible mistake in the restatement (a wrong
table entry, a dropped term, a wrong sign or index, a transposed operand)
fails: known answers of the reference's own tests, closed forms, brute force
evaluations on tiny inputs and finite differences.
"""

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch
from scipy.signal import butter, sosfilt, tf2sos

from oracle import pesq_oracle as O

TABLES = json.loads((Path(__file__).parent / "golden" / "tables.json").read_text())


def test_tables_match_golden():
    c = O.constants()
    counts = TABLES["nr_of_hz_bands_per_bark_band_16k"]
    assert sum(counts) == 256
    # tests/test_fbank.py:5-11: every bin in exactly one band, band sizes as tabled
    assert torch.equal(c["fbank"].sum(0), torch.ones(256, dtype=torch.float64))
    assert torch.equal(c["fbank"].sum(1), torch.tensor(counts, dtype=torch.float64))
    np.testing.assert_array_equal(c["threshs"].numpy(), np.array(TABLES["abs_thresh_power_16k"]))
    np.testing.assert_array_equal(c["width_bark"].numpy(), np.array(TABLES["width_of_band_bark_16k"]))
    np.testing.assert_allclose(
        c["corr"].numpy(),
        np.array(TABLES["pow_dens_correction_factor_16k"]) * TABLES["Sp_16k"],
        rtol=1e-15,
    )
    # Zwicker exponents: clamp(6 / (c + 2), 1, 2)^0.15 * 0.23, float32 values
    centre = np.array(TABLES["centre_of_band_bark_16k"])
    want = np.clip(6 / (centre + 2), 1, 2) ** 0.15 * 0.23
    np.testing.assert_allclose(c["exp"].numpy(), want, rtol=1e-6)
    assert c["exp"].float().double().equal(c["exp"])


def test_power_filter_is_the_float32_butterworth():
    c = O.constants()
    b, a = butter(5, [325, 3250], fs=16000, btype="band")
    assert c["power_b"].numel() == 11 and c["power_a"].numel() == 11
    np.testing.assert_array_equal(c["power_b"].numpy(), np.float32(b).astype(np.float64))
    np.testing.assert_array_equal(c["power_a"].numpy(), np.float32(a).astype(np.float64))


def _recursion(x, b, a):
    """Textbook difference equation, pure Python, zero initial state."""

    y = np.zeros_like(x)
    for n in range(len(x)):
        acc = sum(b[k] * x[n - k] for k in range(len(b)) if n - k >= 0)
        acc -= sum(a[k] * y[n - k] for k in range(1, len(a)) if n - k >= 0)
        y[n] = acc / a[0]
    return y


@pytest.mark.parametrize("which", ["power", "pre"])
def test_lfilter_matches_difference_equation(which):
    c = O.constants()
    b, a = c[f"{which}_b"].numpy(), c[f"{which}_a"].numpy()
    x = np.random.default_rng(0).standard_normal(300)
    want = _recursion(x, b, a)
    got = O.lfilter64(x[None], b, a)[0]
    assert np.abs(got - want).max() <= 1e-9 * np.abs(want).max()
    # second order sections of the same filter agree too
    np.testing.assert_allclose(sosfilt(tf2sos(b, a), x), want, rtol=0, atol=1e-9 * np.abs(want).max())


def test_lfilter_adjoint_is_time_reversed_filter():
    c = O.constants()
    rng = np.random.default_rng(1)
    x, y = rng.standard_normal(4000), rng.standard_normal(4000)
    b, a = c["power_b"].numpy(), c["power_a"].numpy()
    lhs = float(np.dot(y, O.lfilter64(x[None], b, a)[0]))
    rhs = float(np.dot(O.lfilter64(y[None], b, a, reverse=True)[0], x))
    # the order 10 direct form itself carries ~1e-10 of float64 rounding
    assert abs(lhs - rhs) <= 1e-8 * (abs(lhs) + 1e-30)
    # and a wrong "adjoint" (the forward filter itself) does not pass
    wrong = float(np.dot(O.lfilter64(y[None], b, a)[0], x))
    assert abs(lhs - wrong) > 1e-3 * abs(lhs)


def test_frame_count_known_answers():
    # triton_ops/loss.py:142 pads by N % 256: 128000 -> 499 frames
    assert O.n_frames(128000) == 499
    assert O.n_frames(16000) == 62
    assert O.n_frames(960000) == 3749
    assert O.n_frames(64000) == 249
    # 20000 samples pad by 32 -> 20032 -> 77 frames
    assert O.n_frames(20000) == 77


def test_stft_bark_matches_direct_dft():
    c = O.constants()
    rng = np.random.default_rng(2)
    x = torch.from_numpy(rng.standard_normal((2, 1024)))
    got = O.stft_bark(x, c)
    w = c["window"].numpy()
    k = np.arange(512)
    frames = [x.numpy()[:, 256 * t : 256 * t + 512] * w for t in range(3)]
    power = np.stack([np.abs(f @ np.exp(-2j * np.pi * np.outer(k, np.arange(257)) / 512)) ** 2 for f in frames], 1)
    power[:, :, 0] = 0.0
    want = power[:, :, :256] @ c["fbank"].numpy().T * c["corr"].numpy()
    assert got.shape == (2, 3, 49)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-10, atol=1e-12 * np.abs(want).max())
    # band 0 is the DC bin alone, which is dropped
    assert torch.all(got[:, :, 0] == 0)


@pytest.mark.parametrize(
    "n_fft,hop,win,nbarks,n,n_padded",
    [(256, 100, 256, 32, 1500, 1600), (512, 600, 401, 49, 3000, 3000), (64, 7, 33, 17, 300, 330)],
)
def test_stft_bark_op_matches_direct_dft(n_fft, hop, win, nbarks, n, n_padded):
    """The general operator: any hop, short centred windows, zero padding.

    A direct float64 DFT of every frame (window zero padded to n_fft,
    ``(n_fft - win) // 2`` zeros in front, the ``torch.stft`` rule), DC
    dropped, bins below n_fft / 2 summed per band.  A window that is not
    centred, a wrong hop or a frame count off by one fails it.
    """

    rng = np.random.default_rng(n_fft + hop)
    x = torch.from_numpy(rng.standard_normal((2, n)))
    window = torch.hann_window(win, dtype=torch.float64)
    fbank = O.bark_fbank(n_fft // 2, nbarks)
    corr = torch.from_numpy(rng.uniform(0.5, 2.0, nbarks))
    got = O.stft_bark_op(x, window, fbank, corr, n_fft, hop, n_padded)
    full = np.zeros(n_fft)
    left = (n_fft - win) // 2
    full[left : left + win] = window.numpy()
    xp = np.pad(x.numpy(), ((0, 0), (0, n_padded - n)))
    frames = 1 + (n_padded - n_fft) // hop
    k = np.arange(n_fft)
    basis = np.exp(-2j * np.pi * np.outer(k, np.arange(n_fft // 2)) / n_fft)
    power = np.stack([np.abs((xp[:, hop * t : hop * t + n_fft] * full) @ basis) ** 2 for t in range(frames)], 1)
    power[:, :, 0] = 0.0
    want = power @ fbank.numpy().T * corr.numpy()
    assert got.shape == (2, frames, nbarks)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-10, atol=1e-12 * np.abs(want).max())


@pytest.mark.parametrize("nfreqs", [256, 128, 512, 32])
@pytest.mark.parametrize("nbarks", [49, 32, 17])
def test_bark_fbank_is_a_segmentation(nfreqs, nbarks):
    """``test_triton_spectral.py:176-197``: binary, contiguous, sorted, disjoint.

    At the default geometry the bands are the standard's bin counts.
    """

    fb = O.bark_fbank(nfreqs, nbarks)
    assert torch.all((fb == 0) | (fb == 1))
    prev = 0
    for band in range(nbarks):
        nz = torch.nonzero(fb[band]).flatten()
        if nz.numel() == 0:
            continue
        start, end = int(nz[0]), int(nz[-1]) + 1
        assert end - start == nz.numel() and start >= prev and end <= nfreqs
        prev = end
    if (nfreqs, nbarks) == (256, 49):
        counts = fb.sum(1).numpy().astype(int).tolist()
        assert counts == TABLES["nr_of_hz_bands_per_bark_band_16k"]


def test_stft_bark_gradient_finite_difference():
    c = O.constants()
    x = torch.randn(1, 768, dtype=torch.float64, generator=torch.Generator().manual_seed(3))
    w = torch.randn(1, 2, 49, dtype=torch.float64, generator=torch.Generator().manual_seed(4))
    x.requires_grad_(True)
    (O.stft_bark(x, c) * w).sum().backward()
    for n in (5, 300, 511, 700):
        e = torch.zeros_like(x)
        e[0, n] = 1e-6
        with torch.no_grad():
            fd = ((O.stft_bark(x + e, c) - O.stft_bark(x - e, c)) * w).sum() / 2e-6
        assert abs(float(fd) - float(x.grad[0, n])) <= 1e-6 * max(1.0, abs(float(fd)))


def test_chain_identical_inputs_floor():
    # test_triton_chain.py:365-383: ref == deg gives the 1e-20 floor divided by h
    c = O.constants()
    g = torch.Generator().manual_seed(5)
    ref = c["threshs"] * 10 ** (torch.rand(1, 40, 1, generator=g, dtype=torch.float64) * 6) * (
        0.2 + 2 * torch.rand(1, 40, 49, generator=g, dtype=torch.float64)
    )
    ds, da = O.chain(ref, ref.clone(), c)
    assert float(ds) < 1e-19 and float(da) < 1e-19
    symm, _ = O.frame_distances(ref, ref.clone(), c)
    taer = (ref * (ref > c["threshs"])).sum(2)  # band ratio is 1 for identical inputs
    h = ((taer + 1e5) / 1e7) ** 0.04
    torch.testing.assert_close(symm, (1e-20 / h), rtol=1e-12, atol=0)


def _chain_loops(ref, deg, c):
    """The chain with explicit loops over frames and bands (tiny inputs only)."""

    th, ex, wb = c["threshs"].tolist(), c["exp"].tolist(), c["width_bark"].tolist()
    tw = float(c["total_width"])
    T, K = len(ref), len(ref[0])
    silent = [sum(v for k, v in enumerate(ref[t]) if v > 100 * th[k]) < 1e7 for t in range(T)]
    mr = [sum(ref[t][k] for t in range(T) if not silent[t] and ref[t][k] > 100 * th[k]) / T for k in range(K)]
    md = [sum(deg[t][k] for t in range(T) if not silent[t] and deg[t][k] > 100 * th[k]) / T for k in range(K)]
    r = [min(max((md[k] + 1000) / (mr[k] + 1000), 0.01), 100.0) for k in range(K)]
    er = [[r[k] * ref[t][k] for k in range(K)] for t in range(T)]
    taer = [sum(v for k, v in enumerate(er[t]) if v > th[k]) for t in range(T)]
    tad = [sum(v for k, v in enumerate(deg[t]) if v > th[k]) for t in range(T)]
    f0 = [(taer[t] + 5e3) / (tad[t] + 5e3) for t in range(T)]
    f1 = [f0[0]] + [0.8 * f0[t] + 0.2 * f0[t - 1] for t in range(1, T)]
    fpr = [min(max(v, 3e-4), 5.0) for v in f1]

    def loud(x, k):
        return 0.0 if x <= th[k] else (2 * th[k]) ** ex[k] * ((0.5 + 0.5 * x / th[k]) ** ex[k] - 1) * O.SL

    out_s, out_a = [], []
    for t in range(T):
        s2 = a1 = 0.0
        for k in range(1, K):
            ed = fpr[t] * deg[t][k]
            ld, lr = loud(ed, k), loud(er[t][k], k)
            u = ld - lr
            dist = math.copysign(1.0, u) * max(abs(u) - 0.25 * min(ld, lr), 0.0) if u != 0 else 0.0
            s2 += (wb[k] * dist) ** 2 / tw
            asc = ((ed + 50) / (er[t][k] + 50)) ** 1.2
            asc = 0.0 if asc < 3 else min(asc, 12.0)
            a1 += abs(wb[k] * dist * asc / tw)
        h = ((taer[t] + 1e5) / 1e7) ** 0.04
        out_s.append(min(max(tw * math.sqrt(s2), 1e-20) / h, 45.0))
        out_a.append(min(max(tw * a1, 1e-20) / h, 45.0))

    def sums(v):
        nwin = (T - 20) // 10 + 1
        p = [(sum(v[10 * l + j] ** 6 for j in range(20)) / 20) ** (1 / 6) for l in range(nwin)]
        return math.sqrt(sum(q * q for q in p) / nwin)

    return sums(out_s), sums(out_a)


def test_chain_matches_loop_evaluation():
    c = O.constants()
    g = torch.Generator().manual_seed(6)
    level = 10 ** (torch.rand(1, 31, 1, generator=g, dtype=torch.float64) * 6)
    ref = c["threshs"] * level * (0.2 + 2 * torch.rand(1, 31, 49, generator=g, dtype=torch.float64))
    deg = ref * 10 ** ((torch.rand(1, 31, 49, generator=g, dtype=torch.float64) - 0.5))
    ds, da = O.chain(ref, deg, c)
    ws, wa = _chain_loops(ref[0].tolist(), deg[0].tolist(), c)
    assert abs(float(ds) - ws) <= 1e-12 * ws and abs(float(da) - wa) <= 1e-12 * wa


def test_chain_gradient_finite_difference():
    c = O.constants()
    g = torch.Generator().manual_seed(7)
    level = 10 ** (torch.rand(1, 30, 1, generator=g, dtype=torch.float64) * 5 + 1)
    ref = c["threshs"] * level * (0.5 + torch.rand(1, 30, 49, generator=g, dtype=torch.float64))
    deg = (ref * 10 ** ((torch.rand(1, 30, 49, generator=g, dtype=torch.float64) - 0.5) * 0.6)).requires_grad_(True)
    ds, da = O.chain(ref, deg, c)
    (0.7 * ds + 0.3 * da).sum().backward()
    flat = deg.grad.flatten()
    for idx in torch.topk(flat.abs(), 4).indices.tolist():
        e = torch.zeros_like(flat)
        e[idx] = 1e-7 * abs(float(deg.detach().flatten()[idx]))
        e = e.view_as(deg)
        with torch.no_grad():
            hi = O.chain(ref, deg + e, c)
            lo = O.chain(ref, deg - e, c)
        fd = (0.7 * (hi[0] - lo[0]) + 0.3 * (hi[1] - lo[1])).sum() / (2 * float(e.flatten()[idx]))
        assert abs(float(fd) - float(flat[idx])) <= 1e-4 * abs(float(flat[idx]))


def test_epilogue_known_answers():
    """The epilogue against values evaluated by hand (40-digit decimal
    arithmetic), from the published definitions rather than the reference:
    ITU-T P.862 (02/2001) section 10.2.2 gives the raw score
    ``4.5 - 0.1 d_symm - 0.0309 d_asymm``, and ITU-T P.862.2 (11/2005) maps a
    raw score ``x`` to wideband MOS-LQO ``0.999 + (4.999 - 0.999) / (1 +
    exp(-1.3669 x + 3.8224))``.  (0, 0) is the well known top of the wideband
    scale, 4.644."""

    ds = torch.tensor([0.0, 45.0, 10.0, 2.5], dtype=torch.float64)
    da = torch.tensor([0.0, 45.0, 20.0, 7.5], dtype=torch.float64)
    mos, loss = O.epilogue(ds, da, 0.5)
    want = [4.643888749336258439, 1.012035949416599897, 3.115872494896440961,
            4.365381103103138429]
    torch.testing.assert_close(mos, torch.tensor(want, dtype=torch.float64), rtol=1e-14, atol=0)
    # the loss is factor times the raw score's deficit, 4.5 - x
    torch.testing.assert_close(loss, 0.5 * torch.tensor([0.0, 5.8905, 1.618, 0.48175],
                                                        dtype=torch.float64), rtol=1e-14, atol=0)


# -- the formula constants against the reference's text ----------------------------------


def test_formula_constants_match_the_reference_text():
    """Every constant the oracle's formulas use equals the literal at the
    reference's line (``tables.json`` holds what ``make_tables.py`` parsed
    from the source with ``ast``); the two copies of the chain in the
    reference (``loss.py`` and ``triton_ops/reference.py``) were checked to
    agree when the table was written."""

    parsed = TABLES["formula_constants"]
    assert set(O.FORMULA) == set(parsed)
    for name, value in parsed.items():
        assert O.FORMULA[name] == value, (name, O.FORMULA[name], value,
                                          TABLES["formula_constant_sources"][name])
    # the chain's sl (reference.py:322) is the loudness table's Sl_16k (loudness.py:26)
    assert O.SL == parsed["sl"] == TABLES["Sl_16k"]
    assert (O.WINDOW, O.STRIDE) == (TABLES["psqm_window"], TABLES["psqm_stride"])


def test_oracle_formulas_take_their_constants_from_the_table():
    """No constant is typed inside the oracle's formula functions: every
    numeric literal left there is structural (0, 1, 2 as indices, dims,
    the 1 of a logistic or of ``1 / p``)."""

    import ast
    import inspect

    names = ["total_audible", "silent_frames", "band_means", "band_ratio", "frame_ratio",
             "loudness", "disturbance", "weighted_norm", "asymmetry_factor", "frame_weight",
             "frame_distances", "overlapping_sums", "epilogue", "align_level", "edge_ramp",
             "n_frames", "stft_bark"]
    for name in names:
        tree = ast.parse(inspect.getsource(getattr(O, name)))
        body = tree.body[0].body[1:]  # past the docstring
        for stmt in body:
            for node in ast.walk(stmt):
                if isinstance(node, ast.Constant) and isinstance(node.value, (int, float)):
                    assert node.value in (0, 1, 2), (name, node.value, ast.unparse(stmt))


# -- closed-form consequences of each chain step --------------------------------------------
#
# Each test below evaluates one step of the oracle's chain on inputs whose answer
# follows from the mathematics, and also checks that a plausible misreading
# (a constant changed in ``O.FORMULA``, a mistake planted in the oracle) fails.


def _planted(monkeypatch, **changes):
    for key, value in changes.items():
        monkeypatch.setitem(O.FORMULA, key, value)


def _loudness_laws_hold():
    c = O.constants()
    th, ex = c["threshs"].reshape(1, 1, -1), c["exp"].reshape(1, 1, -1)
    ok = True
    # zero at and below the threshold
    zero = O.loudness(torch.cat([th, 0.5 * th, 0 * th], dim=1), th, ex, O.SL)
    ok &= bool((zero == 0).all())
    # far above the threshold the law tends to sl x^e
    x = th * 1e40
    ok &= bool(((O.loudness(x, th, ex, O.SL) / (O.SL * x**ex)) - 1).abs().max() < 1e-9)
    # just above it, its slope: L(th (1 + 2 d)) ~ sl (2 th)^e e d
    d = 1e-6
    near = O.loudness(th * (1 + 2 * d), th, ex, O.SL) / (O.SL * (2 * th) ** ex * ex * d)
    ok &= bool((near - 1).abs().max() < 1e-5)
    return ok


def test_loudness_laws(monkeypatch):
    assert _loudness_laws_hold()
    for change in ({"loudness_half": 1.0}, {"loudness_threshold_scale": 1.0},
                   {"loudness_one": 0}):
        with monkeypatch.context() as m:
            _planted(m, **change)
            assert not _loudness_laws_hold(), change


def _disturbance_answers(l_ref):
    l_ref = torch.tensor(l_ref, dtype=torch.float64)
    got = [O.disturbance(k * l_ref, l_ref) for k in (2.0, 1.2, 0.5, 1.0, 0.0)]
    want = [0.75 * l_ref, 0 * l_ref, -0.375 * l_ref, 0 * l_ref, -l_ref]
    return all(bool(torch.allclose(g, w, rtol=1e-14, atol=0)) for g, w in zip(got, want))


def test_disturbance_deadzone(monkeypatch):
    """``L_deg = 2 L_ref`` leaves 0.75 L_ref, ``1.2 L_ref`` falls in the dead
    zone, ``0.5 L_ref`` leaves -0.375 L_ref, a silent deg leaves -L_ref; the
    rule is antisymmetric."""

    l_ref = [1.0, 3.5, 1e-3]
    assert _disturbance_answers(l_ref)
    a = torch.tensor([0.3, 2.0, 5.0], dtype=torch.float64)
    b = torch.tensor([1.0, 1.1, 0.2], dtype=torch.float64)
    assert torch.equal(O.disturbance(a, b), -O.disturbance(b, a))
    with monkeypatch.context() as m:
        _planted(m, deadzone=0.2)
        assert not _disturbance_answers(l_ref)


def _psqm_answers():
    v = 3.0
    root = 0.6069622310029172  # 20^(-1/6)
    ok = True
    for frames, t, windows_in, nwin in ((50, 15, 2, 4), (50, 5, 1, 4), (50, 45, 1, 4),
                                        (49, 45, 0, 3), (40, 20, 2, 3), (40, 9, 1, 3)):
        x = torch.zeros(1, frames, dtype=torch.float64)
        x[0, t] = v
        want = v * root * math.sqrt(windows_in / nwin)
        ok &= abs(float(O.overlapping_sums(x)) - want) <= 1e-14 * v
    const = torch.full((1, 57), 7.25, dtype=torch.float64)
    ok &= abs(float(O.overlapping_sums(const)) - 7.25) <= 1e-13
    return ok


def test_overlapping_sums_single_frame(monkeypatch):
    """One non-zero frame v: each window holding it has the 6th power mean
    ``v 20^(-1/6)``, the others 0, so the RMS over ``nwin`` windows is
    ``v 20^(-1/6) sqrt(m / nwin)`` for a frame inside m windows (windows of 20
    frames at stride 10: frame 15 is in two, frame 5 in one, frame 45 of 49
    in none); a constant sequence gives the constant."""

    assert _psqm_answers()
    for change in ({"psqm_power": 4}, {"psqm_stride": 5}, {"psqm_window": 10}):
        with monkeypatch.context() as m:
            _planted(m, **change)
            monkeypatch.setattr(O, "WINDOW", O.FORMULA["psqm_window"])
            monkeypatch.setattr(O, "STRIDE", O.FORMULA["psqm_stride"])
            assert not _psqm_answers(), change
            monkeypatch.setattr(O, "WINDOW", 20)
            monkeypatch.setattr(O, "STRIDE", 10)


def _silence_and_means_answers():
    c = O.constants()
    th = c["threshs"]
    T = 8
    spec = torch.zeros(1, T, 49, dtype=torch.float64)
    spec[0, :, 30] = 2e7          # frames of 2e7 above 100 th: not silent
    spec[0, 4:, 30] = 0.5e7       # half of them at 0.5e7: silent
    spec[0, :, 20] = 50 * th[20]  # audible, but below 100 th: never in a mean
    spec[0, 1, 0] = 99 * th[0]    # 5e9 of energy below 100 th_0: does not count
    silent = O.silent_frames(spec, th)
    ok = silent.tolist() == [[False] * 4 + [True] * 4]
    # a frame whose only energy is band 0 at 99 th_0 (about 5.1e9) is silent
    lone = torch.zeros(1, 2, 49, dtype=torch.float64)
    lone[0, 0, 0] = 99 * th[0]
    lone[0, 1, 0] = 101 * th[0]
    ok &= O.silent_frames(lone, th).tolist() == [[True, False]]
    means = O.band_means(spec, th, silent)
    # the mean over all 8 frames of the 4 non-silent frames' 2e7: 1e7
    ok &= abs(float(means[0, 30]) - 1e7) <= 1e-6
    ok &= float(means[0, 20]) == 0.0 and float(means[0, 0]) == 0.0
    return ok


def test_silent_frames_and_band_means(monkeypatch):
    """A frame is silent when its reference energy in bands above 100 times
    their threshold is below 1e7; the band means sum the non-silent frames'
    powers above 100 th and divide by all frames."""

    assert _silence_and_means_answers()
    for change in ({"silent_energy": 1e6}, {"mean_threshold_factor": 1.0},
                   {"silent_threshold_factor": 1.0}):
        with monkeypatch.context() as m:
            _planted(m, **change)
            assert not _silence_and_means_answers(), change


def _band_ratio_answers():
    t = lambda v: torch.tensor([v], dtype=torch.float64)  # noqa: E731
    got = [float(O.band_ratio(t(mr), t(md))) for mr, md in
           ((0.0, 0.0), (1000.0, 3000.0), (1e9, 0.0), (0.0, 1e9), (9000.0, 0.0))]
    return got == [1.0, 2.0, 0.01, 100.0, 0.1]


def test_band_ratio_known_answers(monkeypatch):
    assert _band_ratio_answers()
    for change in ({"band_ratio_offset": 100}, {"band_ratio_min": 0.001},
                   {"band_ratio_max": 1000.0}):
        with monkeypatch.context() as m:
            _planted(m, **change)
            assert not _band_ratio_answers(), change


def _frame_ratio_answers():
    # raw ratios (taer + 5e3) / (tad + 5e3): 2, 1, 0.25, 1e-8, 1e-8, 100
    taer = torch.tensor([[5e3, 7e3, 0.0, 0.0, 0.0, 4.95e5]], dtype=torch.float64)
    tad = torch.tensor([[0.0, 7e3, 15e3, 5e11 - 5e3, 5e11 - 5e3, 0.0]], dtype=torch.float64)
    # smoothed 0.8 f_t + 0.2 f_(t-1) for t > 0, clamped to [3e-4, 5]
    want = torch.tensor([[2.0, 1.2, 0.4, 0.05 + 0.8e-8, 3e-4, 5.0]], dtype=torch.float64)
    return bool(torch.allclose(O.frame_ratio(taer, tad), want, rtol=1e-12, atol=0))


def test_frame_ratio_known_answers(monkeypatch):
    assert _frame_ratio_answers()
    for change in ({"frame_smooth_current": 0.2, "frame_smooth_previous": 0.8},
                   {"frame_ratio_offset": 1e3}, {"frame_ratio_min": 3e-3},
                   {"frame_ratio_max": 10.0}):
        with monkeypatch.context() as m:
            _planted(m, **change)
            assert not _frame_ratio_answers(), change


def _asymmetry_answers():
    er = torch.zeros(5, dtype=torch.float64)
    ed = torch.tensor([75.0, 74.0, 350.0, 0.0, 200.0], dtype=torch.float64)
    want = torch.tensor([3.002811084953578,  # 2.5^1.2, above the cut of 3
                         0.0,                # 2.48^1.2 = 2.974, below it
                         12.0,               # 8^1.2 = 12.126, capped
                         0.0,                # 1
                         6.898648307306074], dtype=torch.float64)  # 5^1.2
    return bool(torch.allclose(O.asymmetry_factor(ed, er), want, rtol=1e-14, atol=0))


def test_asymmetry_factor_known_answers(monkeypatch):
    assert _asymmetry_answers()
    for change in ({"asymm_exponent": 1.0}, {"asymm_offset": 5.0}, {"asymm_cut": 2.9},
                   {"asymm_cap": 20.0}):
        with monkeypatch.context() as m:
            _planted(m, **change)
            assert not _asymmetry_answers(), change


def _frame_weight_answers():
    taer = torch.tensor([0.0, 9.9e6, 1e7 * 2**25 - 1e5], dtype=torch.float64)
    # h(0) = 0.01^0.04: the 0.83175 of the identical-input floor at
    # test_triton_chain.py:725-750; h(9.9e6) = 1; h(2^25 1e7 - 1e5) = 2
    want = torch.tensor([0.8317637711026710, 1.0, 2.0], dtype=torch.float64)
    return bool(torch.allclose(O.frame_weight(taer), want, rtol=1e-14, atol=0))


def test_frame_weight_known_answers(monkeypatch):
    assert _frame_weight_answers()
    for change in ({"h_offset": 1e4}, {"h_scale": 1e6}, {"h_exponent": 0.4}):
        with monkeypatch.context() as m:
            _planted(m, **change)
            assert not _frame_weight_answers(), change


def _norm_answers():
    c = O.constants()
    wb, tw = c["width_bark"], float(c["total_width"])
    ok = abs(tw - sum(TABLES["width_of_band_bark_16k"][1:])) <= 1e-12 * tw
    d = torch.zeros(1, 1, 49, dtype=torch.float64)
    d[0, 0, 17] = -2.5
    # one band: sqrt(W) w_k |d| for p = 2, w_k |d| for p = 1
    ok &= abs(float(O.weighted_norm(d, wb, tw, 2)) - math.sqrt(tw) * float(wb[17]) * 2.5) <= 1e-12
    ok &= abs(float(O.weighted_norm(d, wb, tw, 1)) - float(wb[17]) * 2.5) <= 1e-12
    d[0, 0, 30] = 1.5
    two = math.sqrt(tw) * math.hypot(float(wb[17]) * 2.5, float(wb[30]) * 1.5)
    ok &= abs(float(O.weighted_norm(d, wb, tw, 2)) - two) <= 1e-12
    # band 0 is left out of both norms
    z = torch.zeros(1, 1, 49, dtype=torch.float64)
    z[0, 0, 0] = 9.0
    ok &= float(O.weighted_norm(z, wb, tw, 2)) == 0.0 and float(O.weighted_norm(z, wb, tw, 1)) == 0.0
    return ok


def test_weighted_norms_absolute_scale(monkeypatch):
    """``W ||w d / W^(1/p)||_p`` over bands 1..48: a single band k gives
    ``sqrt(W) w_k |d|`` (p = 2) and ``w_k |d|`` (p = 1); band 0 is excluded;
    W is the sum of the widths of bands 1..48."""

    assert _norm_answers()
    with monkeypatch.context() as m:
        _planted(m, norm_first_band=0)
        assert not _norm_answers()


def _single_band_distances(k, ref_level, deg_level, frames=40):
    ref = torch.zeros(1, frames, 49, dtype=torch.float64)
    deg = torch.zeros(1, frames, 49, dtype=torch.float64)
    ref[:, :, k] = ref_level
    deg[:, :, k] = deg_level
    return [float(v) for v in O.chain(ref, deg)]


@pytest.mark.parametrize("k", [10, 25, 40])
def test_chain_single_band_absolute_distances(k):
    """Constant single-band spectra through the whole chain (every frame the
    same, so the overlapping sums return the frame value):

    * ref = A >= 1e7 in band k, deg = 0: the band ratio is
      ``max(1000 / (A + 1000), 0.01)``, equ_ref = ratio A, the disturbance is
      ``-L(equ_ref)``, so ``d_symm = sqrt(W) w_k L(equ_ref) / h(equ_ref)`` and
      the asymmetry factor ``(50 / (equ_ref + 50))^1.2 < 3`` leaves
      ``d_asymm = 1e-20 / h(equ_ref)``;
    * ref = 0 (every frame silent, band ratio 1), deg = B in band k: the frame
      ratio is ``5e3 / (B + 5e3)``, equ_deg = that times B, h = h(0), and
      ``d_symm = sqrt(W) w_k L(equ_deg) / h(0)``,
      ``d_asymm = w_k L(equ_deg) ((equ_deg + 50) / 50)^1.2 / h(0)``.
    """

    c = O.constants()
    th, ex = c["threshs"][k], c["exp"][k]
    wk, tw = float(c["width_bark"][k]), float(c["total_width"])
    loud = lambda x: float(O.loudness(torch.tensor(x, dtype=torch.float64), th, ex, O.SL))  # noqa: E731
    h = lambda taer: (taer + 1e5) / 1e7  # noqa: E731

    a = 3e7
    equ_ref = max(1000.0 / (a + 1000.0), 0.01) * a
    ds, da = _single_band_distances(k, a, 0.0)
    assert abs(ds - math.sqrt(tw) * wk * loud(equ_ref) / h(equ_ref) ** 0.04) <= 1e-12 * ds
    assert abs(da - 1e-20 / h(equ_ref) ** 0.04) <= 1e-12 * da

    b = 5000.0 * 200.0 / 4800.0  # equ_deg = 200: an asymmetry factor of 5^1.2
    equ_deg = 5e3 / (b + 5e3) * b
    ds, da = _single_band_distances(k, 0.0, b)
    h0 = h(0.0) ** 0.04
    assert abs(ds - math.sqrt(tw) * wk * loud(equ_deg) / h0) <= 1e-12 * ds
    asc = ((equ_deg + 50.0) / 50.0) ** 1.2
    assert 3.0 < asc < 12.0
    assert abs(da - wk * loud(equ_deg) * asc / h0) <= 1e-12 * da


def _signals(batch, n, seed):
    from bench import speech_like_pair

    ref, deg = speech_like_pair(batch, n, seed=seed, noise=0.1)
    return torch.from_numpy(ref).double(), torch.from_numpy(deg).double()


def test_pipeline_scale_invariance_and_batch_independence():
    ref, deg = _signals(3, 8000, 8)
    ds, da = O.pipeline(ref, deg)
    ds2, da2 = O.pipeline(ref * 7.5, deg * 1e-3)
    torch.testing.assert_close(ds2, ds, rtol=1e-9, atol=0)
    torch.testing.assert_close(da2, da, rtol=1e-9, atol=0)
    one = O.pipeline(ref[1:2], deg[1:2])
    assert abs(float(one[0]) - float(ds[1])) <= 1e-12 * float(ds[1])


def test_pipeline_identical_signals_zero_loss():
    # test_torch.py:18-27: loss(ref, ref) <= 1e-20 (here: the floor / h)
    ref, _ = _signals(2, 8000, 9)
    ds, da = O.pipeline(ref, ref.clone())
    _, loss = O.epilogue(ds, da, 1.0)
    assert torch.all(loss < 1e-19) and torch.all(loss > 0)


@pytest.mark.parametrize(
    "orig,new,width,total",
    # width_total known answers of test_triton_resample.py:13,177-181,685-686
    [(44100, 16000, 17, 475), (48000, 16000, 19, 41), (8000, 16000, 7, 15)],
)
def test_resample_kernel_shape_known_answers(orig, new, width, total):
    kernel, w = O.sinc_resample_kernel(orig, new)
    g = math.gcd(orig, new)
    assert w == width and kernel.shape == (new // g, total)
    assert kernel.dtype == torch.float32


@pytest.mark.parametrize("orig,new", [(44100, 16000), (48000, 16000), (8000, 16000)])
def test_resample_kernel_properties(orig, new):
    kernel, width = O.sinc_resample_kernel(orig, new)
    k = kernel.double()
    # DC gain: every phase of a low pass interpolator sums to ~1 (rolloff 0.99 + window)
    assert torch.all((k.sum(1) - 1).abs() < 2e-3)
    # phase 0 is symmetric about the tap at offset `width`
    phase0 = k[0]
    g = math.gcd(orig, new)
    centre = width
    half = min(centre, phase0.shape[0] - 1 - centre)
    torch.testing.assert_close(phase0[centre - half : centre], phase0[centre + 1 : centre + half + 1].flip(0), rtol=0, atol=1e-6)
    assert float(phase0[centre]) == pytest.approx(min(orig, new) // g * 0.99 / (orig // g), rel=1e-6)


def test_resample_lengths_and_identity():
    # output length = float32 ceil of new * n / orig (test_triton_resample.py:620-647)
    assert O.resample_length(176400, 44100, 16000) == 64000
    assert O.resample_length(192000, 48000, 16000) == 64000
    assert O.resample_length(1000, 48000, 16000) == 334
    assert O.resample_length(0, 48000, 16000) == 0
    x = torch.randn(2, 100, dtype=torch.float64)
    assert O.resample(x, 16000) is x
    # a pure tone below the cut-off survives 48 -> 16 kHz resampling
    t = torch.arange(48000, dtype=torch.float64) / 48000
    tone = torch.sin(2 * math.pi * 1000 * t)[None]
    out = O.resample(tone, 48000)
    want = torch.sin(2 * math.pi * 1000 * torch.arange(16000, dtype=torch.float64) / 16000)
    assert (out[0, 200:-200] - want[200:-200]).abs().max() < 2e-3


# -- resampler: brute force over the continuous kernel ----------------------------


def _brute_force_resample(x, orig_freq, new_freq, float32_rounding, lpw=6, rolloff=0.99):
    """``y[m] = sum_n x[n] h((n / orig - m / new) base) base / orig``, one output at a time.

    ``h(t) = sinc(pi t) cos(pi t / (2 lpw))^2`` on ``|t| <= lpw`` is torchaudio's
    published Hann windowed sinc; ``base = min(orig, new) rolloff`` with the
    rates reduced by their gcd; the input is zero outside ``[0, len(x))``.  No
    filter bank, convolution or reshape: every output walks the input samples
    its kernel covers.  ``float32_rounding`` applies the two roundings
    torchaudio's tap table has (the output phase ``-j / new`` formed in
    float32, the taps stored in float32); without it everything is float64.
    """

    g = math.gcd(orig_freq, new_freq)
    orig, new = orig_freq // g, new_freq // g
    base = min(orig, new) * rolloff
    y = np.zeros(O.resample_length(len(x), orig_freq, new_freq))
    for m in range(len(y)):
        lo = max(math.floor((m / new - lpw / base) * orig) - 1, 0)
        hi = min(math.ceil((m / new + lpw / base) * orig) + 1, len(x) - 1)
        n = np.arange(lo, hi + 1)
        if float32_rounding:
            j, frame = m % new, m // new
            t = (float(np.float32(-j / new)) + (n - frame * orig) / orig) * base
        else:
            t = (n * new - m * orig) / (orig * new) * base
        t = np.clip(t, -lpw, lpw)
        window = np.cos(t * math.pi / lpw / 2) ** 2
        arg = t * math.pi
        sinc = np.where(arg == 0, 1.0, np.sin(arg) / np.where(arg == 0, 1.0, arg))
        taps = sinc * window * (base / orig)
        if float32_rounding:
            taps = taps.astype(np.float32).astype(np.float64)
        y[m] = np.dot(x[n], taps)
    return y


@pytest.mark.parametrize(
    "orig,new,n",
    [(44100, 16000, 1500), (22050, 16000, 1000), (48000, 16000, 600), (13, 7, 300), (7, 13, 300)],
)
def test_resample_matches_brute_force_over_the_continuous_kernel(orig, new, n):
    """Pins the phase convention (sign of ``-j / new``), the phase interleave of
    the output, the ``(width, width + orig)`` padding and the tap support of
    the oracle's polyphase form: with torchaudio's two float32 roundings the
    per-output sum agrees to rounding; in plain float64 it agrees to the size
    of those roundings."""

    x = np.random.default_rng(orig + 3 * new).standard_normal(n)
    got = O.resample(torch.from_numpy(x)[None], orig, new)[0].numpy()
    scale = np.abs(got).max()
    exact = _brute_force_resample(x, orig, new, float32_rounding=True)
    assert got.shape == exact.shape
    assert np.abs(got - exact).max() <= 1e-12 * scale
    plain = _brute_force_resample(x, orig, new, float32_rounding=False)
    assert np.abs(got - plain).max() <= 2e-5 * scale


def _multitone_error(fs, resample):
    """Largest deviation of resampled pass-band tones from the same tones sampled at 16 kHz."""

    n = fs // 2
    tones = [(300.0, 0.3, 0.1), (1000.0, 1.0, 1.3), (2200.0, 0.5, 2.0), (3400.0, 0.7, -0.7)]
    t = np.arange(n) / fs
    x = sum(a * np.sin(2 * math.pi * f * t + p) for f, a, p in tones)
    y = resample(torch.from_numpy(x)[None], fs)[0].numpy()
    m = np.arange(len(y)) / 16000
    want = sum(a * np.sin(2 * math.pi * f * m + p) for f, a, p in tones)
    return float(np.abs(y - want)[400:-400].max())


@pytest.mark.parametrize("fs", [44100, 22050, 48000, 32000])
def test_resample_multitone_passband(fs):
    """Four tones of 0.3 - 3.4 kHz (amplitude sum 2.5) keep amplitude and phase to
    1e-3 of full scale (the measured pass-band ripple is 1.1e-3 in absolute
    units); a wrong phase sign or interleave moves samples by a fraction of an
    input period and errs by 0.1 or more."""

    assert _multitone_error(fs, O.resample) < 2.5e-3


def test_resample_multitone_detects_a_wrong_interleave(monkeypatch):
    """The multitone check fails on a planted mistake: the phases of the filter
    bank in reverse order (the sign of the phase term flipped, modulo one
    sample)."""

    real = O.sinc_resample_kernel

    def flipped(*args, **kwargs):
        kernel, width = real(*args, **kwargs)
        return kernel.flip(0).contiguous(), width

    monkeypatch.setattr(O, "sinc_resample_kernel", flipped)
    assert _multitone_error(44100, O.resample) > 0.05


# -- chain: clamp known answers ---------------------------------------------------


def _single_band(k, ref_level, deg_level, frames=40):
    """Constant spectra with energy in band ``k`` only (float32 values, as the kernels get them).

    All other bands are exactly zero, so they have no loudness and no
    disturbance, every frame is the same (the overlapping 6th-power means of a
    constant are that constant), and both weighted norms reduce to the single
    term of band ``k``: ``symm = sqrt(W) w_k |d_k| / h`` and
    ``asymm = w_k |d_k| asc_k / h`` with ``W`` the total band width.
    """

    ref = torch.zeros(1, frames, 49, dtype=torch.float64)
    deg = torch.zeros(1, frames, 49, dtype=torch.float64)
    ref[:, :, k] = ref_level
    deg[:, :, k] = deg_level
    return ref.float().double(), deg.float().double()


A_LEVEL = 2e7  # one band above 1e7 and above 100 x its threshold: no frame is silent


def test_chain_45_cap():
    """deg = 1e7 ref in band 40: every frame's disturbances exceed 45, both distances are 45."""

    ds, da = O.chain(*_single_band(40, A_LEVEL, 1e7 * A_LEVEL))
    assert abs(float(ds) - 45.0) < 1e-12 and abs(float(da) - 45.0) < 1e-12


@pytest.mark.parametrize("k", [10, 25, 40])
def test_chain_band_ratio_floor_and_asymmetry_cut(k):
    """deg = 1e-6 ref: the degraded band is below 100 x threshold (no band mean),
    so the band ratio 1000 / (A + 1000) clamps at 0.01 and taer = 0.01 A; the
    equalised degraded band is quieter than the reference, the asymmetry
    factor is below 3 and is cut, and the asymmetric distance is the 1e-20
    floor over h = ((0.01 A + 1e5) / 1e7)^0.04.  The symmetric one is not."""

    ref, deg = _single_band(k, A_LEVEL, 1e-6 * A_LEVEL)
    ds, da = O.chain(ref, deg)
    h = ((0.01 * float(ref[0, 0, k]) + 1e5) / 1e7) ** 0.04
    assert abs(float(da) * h / 1e-20 - 1.0) < 1e-12
    assert 1.0 < float(ds) < 45.0


@pytest.mark.parametrize("k", [10, 25])
@pytest.mark.parametrize("louder", [1.5e6, 3e6])
def test_chain_upper_clamps_and_asymmetry_factor(k, louder):
    """deg = q ref with q >= 1.5e6: the band ratio clamps at 100 (equ_ref = 100 A)
    and the frame ratio (100 A + 5e3) / (q A + 5e3) at 3e-4 (equ_deg = 3e-4 q A),
    so asc = ((3e-4 q A + 50) / (100 A + 50))^1.2, 6.1 at q = 1.5e6 and 14.0,
    capped at 12, at q = 3e6; with one band the distances' ratio is
    asc / sqrt(W), whatever the loudness of the band."""

    ref, deg = _single_band(k, A_LEVEL, louder * A_LEVEL)
    ds, da = O.chain(ref, deg)
    c = O.constants()
    a, b = float(ref[0, 0, k]), float(deg[0, 0, k])
    asc = min(((3e-4 * b + 50) / (100 * a + 50)) ** 1.2, 12.0)
    assert (asc == 12.0) == (louder == 3e6)
    assert float(ds) < 45.0 and float(da) < 45.0
    assert abs(float(da / ds) / (asc / math.sqrt(float(c["total_width"]))) - 1.0) < 1e-12


@pytest.mark.parametrize("k", [10, 25, 40])
def test_chain_frame_ratio_cap(k):
    """deg at th_k / 6 in band k: taer = 0.01 A, tad = 0 (below threshold), the frame
    ratio (0.01 A + 5e3) / 5e3 = 41 clamps at 5, and 5 deg <= th_k has no
    loudness, exactly like deg = 0: both give the same distances.  Without the
    clamp (or with one above 6) the degraded band would be audible; at th_k / 3
    (5 deg > th_k) it is, and the distances differ."""

    th = float(O.constants()["threshs"][k])
    quiet = O.chain(*_single_band(k, A_LEVEL, th / 6))
    silent = O.chain(*_single_band(k, A_LEVEL, 0.0))
    assert float(quiet[0]) == float(silent[0]) and float(quiet[1]) == float(silent[1])
    audible = O.chain(*_single_band(k, A_LEVEL, th / 3))
    assert float(audible[0]) != float(silent[0])


@pytest.mark.parametrize("deg_scale", [1.0, 100.0])
def test_chain_exact_threshold_values(deg_scale):
    """``test_triton_chain.py:725-750``: ref = threshs exactly has no loudness (the
    ``x > th`` branch is off) and every frame is silent; deg = threshs or 100
    threshs (frame ratio clamped at 3e-4) has none either, so both distances
    are the floor 1e-20 / h with h = ((0 + 1e5) / 1e7)^0.04 = 0.83175.  (The
    float64 thresholds themselves: their float32 roundings lie above some of
    them, which turns the branch on in those bands.)"""

    th = O.constants()["threshs"].reshape(1, 1, -1)
    ref = th.expand(2, 62, 49).contiguous()
    deg = (th * deg_scale).expand(2, 62, 49).contiguous()
    ds, da = O.chain(ref, deg)
    h = (1e5 / 1e7) ** 0.04
    assert abs(h - 0.83175) < 5e-5  # the reference quotes five digits
    torch.testing.assert_close(ds, torch.full_like(ds, 1e-20 / h), rtol=1e-12, atol=0)
    torch.testing.assert_close(da, torch.full_like(da, 1e-20 / h), rtol=1e-12, atol=0)
