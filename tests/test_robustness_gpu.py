"""The reference's robustness contract on the GPU.

* which kernels a step launches (``tests/test_triton_iir.py:528-554``): the
  loss's forward and backward run only the library's kernels, exactly the
  ones ``pesq_pipeline_kernels`` lists, once each;
* no scratch buffer is read before it is written
  (``tests/test_triton_chain.py:601-621``, ``test_triton_resample.py:592-616``,
  ``test_triton_iir.py:520``): the caching allocator is filled with NaN or
  -1e30 first, and every result must stay finite and bitwise equal;
* a randomised sweep over shapes, levels and degradation types against the
  float64 oracle (``tests/test_triton_loss.py:374-406``), at the north star
  bound ``1e-5``;
* the test signals are not clamp saturated (``test_triton_loss.py:194-213``);
* the perceptual chain on random spectra (``test_triton_chain.py:528-550``)
  and at its clamps (``:332-362,725-750``): the same inputs as the oracle's
  known-answer tests in ``test_oracle.py``, forward and gradients against
  float64.  Chain budgets: 1e-6 forward and 1e-5 gradients, relative to the
  largest float64 magnitude (the reference's are 6e-6 / 3e-5; the kernels
  evaluate the chain in float64, what remains is float32 I/O rounding).
"""

import math
import random

import numpy as np
import pytest
import torch

from bench import speech_like_pair, synthetic_config
from kernel_trace import launched_kernels, library_kernels
from oracle import pesq_oracle as O
from torch_pesq import PesqLoss, PesqLossTriton, _lib
from torch_pesq.hip_ops.chain import HipPesqChain
from torch_pesq.hip_ops.resample import HipResample

pytestmark = pytest.mark.gpu

F64_RTOL = 1e-5
CHAIN_FWD = 1e-6
CHAIN_GRAD = 1e-5


@pytest.fixture(scope="module")
def model():
    return PesqLossTriton(0.5, sample_rate=16000).cuda()


@pytest.fixture(scope="module")
def chain():
    base = PesqLoss(1.0, sample_rate=16000)
    return HipPesqChain(base.loudness.threshs, base.loudness.exp, base.fbank.width_bark,
                        base.fbank.total_width).cuda()


# -- kernel set -----------------------------------------------------------------


@pytest.mark.parametrize("batch,samples", [(8, 128000), (2, 24000)])
def test_only_library_kernels_touch_the_data(model, batch, samples):
    ref, deg = speech_like_pair(batch, samples, seed=21, noise=0.1)
    r = torch.from_numpy(ref).cuda()
    d = torch.from_numpy(deg).cuda().requires_grad_(True)
    upstream = torch.linspace(0.5, 1.5, batch, device="cuda")

    def step():
        return torch.autograd.grad(model(r, d), d, upstream)

    step()
    _, kernels = launched_kernels(step)
    want = library_kernels(batch, samples, _lib.GRAD_DEG, False)
    want += library_kernels(batch, samples, _lib.GRAD_DEG, True)
    assert kernels == {name: 1 for name in want}, sorted(kernels)


def test_sum_and_implicit_gradient_add_only_pytorch_glue(model):
    """``grad(loss.sum(), deg)``: PyTorch's own reduction, the ones fill of the
    implicit gradient and the contiguous copy of its broadcast (three [B]
    sized kernels) join the library's eight."""

    ref, deg = speech_like_pair(8, 128000, seed=22, noise=0.1)
    r = torch.from_numpy(ref).cuda()
    d = torch.from_numpy(deg).cuda().requires_grad_(True)

    def step():
        return torch.autograd.grad(model(r, d).sum(), d)

    step()
    _, kernels = launched_kernels(step)
    ours = set(library_kernels(8, 128000, _lib.GRAD_DEG, False))
    ours |= set(library_kernels(8, 128000, _lib.GRAD_DEG, True))
    assert ours <= set(kernels)
    glue = {k: n for k, n in kernels.items() if k not in ours}
    assert sum(glue.values()) <= 3, glue
    assert all(k.startswith("at::native::") for k in glue), glue


# -- uninitialised reads ------------------------------------------------------------


def _poison(value, numels):
    """Fill the caching allocator with ``value`` in blocks of the given sizes."""

    torch.cuda.synchronize()
    blocks = []
    for numel in numels:
        blocks.extend(torch.full((int(numel),), value, device="cuda") for _ in range(4))
    torch.cuda.synchronize()
    del blocks


def _generic_sizes():
    return [1, 8, 64, 512, 4096, 32768, 262144, 1048576]


@pytest.mark.parametrize("poison", [float("nan"), -1e30])
@pytest.mark.parametrize(
    "batch,samples",
    # small grid (lane states, windowed block starts, the backward's level
    # alignment aggregate in the STFT forward); 293 blocks per row (windowed
    # block starts, the backward's own aggregate launch); 320 x 63 forward and
    # 160 x 63 backward scan wavefronts (lane states recomputed, prefix
    # kernel) with 2560 frame tiles (four frames per wavefront)
    [(2, 24000), (3, 300000), (160, 64000)],
)
def test_no_uninitialised_reads_pipeline(model, poison, batch, samples):
    ref, deg = speech_like_pair(batch, samples, seed=23, noise=0.1)
    r = torch.from_numpy(ref).cuda().requires_grad_(True)
    d = torch.from_numpy(deg).cuda().requires_grad_(True)
    w = torch.linspace(-1.0, 2.0, batch, device="cuda")

    def run():
        out = model._run(r, d)
        grads = torch.autograd.grad(out[3], [r, d], grad_outputs=w)
        return [o.detach().clone() for o in out] + [g.clone() for g in grads]

    clean = run()
    lib = _lib.library()
    fwd = _lib.size_query(lib.pesq_pipeline_forward_workspace, batch, samples, 3)
    bwd = _lib.size_query(lib.pesq_pipeline_backward_workspace, batch, samples, 3)
    _poison(poison, [fwd // 4, bwd // 4, batch * samples, batch] + _generic_sizes())
    dirty = run()
    for name, a, b in zip(("d_symm", "d_asymm", "mos", "loss", "g_ref", "g_deg"), clean, dirty):
        assert torch.isfinite(b).all(), f"{name}: a scratch buffer is read before it is written"
        assert torch.equal(a, b), name


@pytest.mark.parametrize("poison", [float("nan"), -1e30])
def test_no_uninitialised_reads_operators(chain, poison):
    g = torch.Generator().manual_seed(24)
    x = torch.randn(3, 40001, generator=g).cuda()
    base = PesqLoss(1.0, sample_rate=16000).cuda()
    iir, stft = base.power_iir, base.spectral
    rs = HipResample(44100, 16000).cuda()
    spectra = 10 ** (torch.rand(3, 63, 49, generator=g) * 6) * 100.0
    ref_b, deg_b = spectra.cuda(), (spectra * (0.5 + torch.rand(3, 63, 49, generator=g))).cuda()

    def run():
        outs = []
        for fn, inputs in (
            (iir, [x]),
            (rs, [x]),
            (lambda s: stft(s), [x * 1000.0]),
            (lambda a, b: chain(a, b), [ref_b, deg_b]),
        ):
            leaves = [t.clone().requires_grad_(True) for t in inputs]
            out = fn(*leaves)
            out = out if isinstance(out, tuple) else (out,)
            ups = [torch.linspace(0.5, 1.5, o.numel(), device="cuda").view_as(o) for o in out]
            grads = torch.autograd.grad(out, leaves, grad_outputs=ups)
            outs += [o.detach().clone() for o in out] + [gr.clone() for gr in grads]
        return outs

    clean = run()
    _poison(poison, [o.numel() for o in clean] + _generic_sizes())
    dirty = run()
    for i, (a, b) in enumerate(zip(clean, dirty)):
        assert torch.isfinite(b).all(), i
        assert torch.equal(a, b), i


# -- randomised sweep against float64 --------------------------------------------


@pytest.mark.parametrize("seed", range(6))
def test_random_signals_match_float64(model, seed):
    """Random batch (1..5), length (16000..40000), level (1e-2..1e2) and
    degradation (noisy, heavily degraded, clipped), against the oracle."""

    rng = np.random.default_rng(1000 + seed)
    batch = int(rng.integers(1, 6))
    samples = int(rng.integers(16000, 40000))
    level = 10 ** (rng.uniform() * 4 - 2)
    ref, deg = speech_like_pair(batch, samples, seed=seed, noise=0.1)
    ref, deg = ref * level, deg * level
    if seed % 3 == 1:
        deg = deg + 2.0 * level * rng.standard_normal((batch, samples))
    elif seed % 3 == 2:
        deg = np.clip(deg, -0.3 * level, 0.3 * level)
    ref, deg = ref.astype(np.float32), deg.astype(np.float32)
    got = model._run(torch.from_numpy(ref).cuda(), torch.from_numpy(deg).cuda())
    ds, da = O.pipeline(torch.from_numpy(ref), torch.from_numpy(deg))
    mos, loss = O.epilogue(ds, da, 0.5)
    for name, g, w in zip(("d_symm", "d_asymm", "mos", "loss"), got, (ds, da, mos, loss)):
        err = float(((g.double().cpu() - w).abs() / w.abs()).max())
        assert err < F64_RTOL, (name, err, batch, samples, level)


@pytest.mark.parametrize("batch,samples,seed", [(2, 16000, 0), (2, 16000, 7), (3, 20000, 13)])
def test_signals_are_not_clamp_saturated(model, batch, samples, seed):
    """The differential tests' signals lie inside the range the loss is used in:
    both distances well inside (1, 42), not pinned to the 45 clamp."""

    ref, deg = speech_like_pair(batch, samples, seed=seed, noise=0.1)
    ds, da = model.raw(torch.from_numpy(ref).cuda(), torch.from_numpy(deg).cuda())
    for d in (ds, da):
        assert torch.all(d > 1.0) and torch.all(d < 42.0), d


def test_config2_symmetric_distance_is_not_clamp_saturated(model):
    """On the BASELINE c2 generator (speech with silent syllables, noise at 0 -
    20 dB SNR) the asymmetric distance sits at or within 0.5 of its 45 clamp
    in every item (noise in the silent syllables), so c2's d_asymm comparison
    says little; the symmetric distance is well inside the range, and the
    speech-like signals above exercise the asymmetric one."""

    ref, deg, _ = synthetic_config(2)
    ds, da = model.raw(torch.from_numpy(ref).cuda(), torch.from_numpy(deg).cuda())
    assert torch.all(ds > 1.0) and torch.all(ds < 42.0), ds
    assert torch.all(da > 44.0) and torch.all(da <= 45.0), da


# -- chain: fuzz and clamps ----------------------------------------------------------


def _spectra(batch, frames, seed, spread=0.5, level=6.0):
    """Log-uniform spectra straddling the thresholds (``test_triton_chain.py:95-113``)."""

    g = torch.Generator().manual_seed(seed)
    th = O.constants()["threshs"].float()
    lv = 10 ** (torch.rand((batch, frames, 1), generator=g) * level)
    tilt = 0.2 + 2.0 * torch.rand((batch, frames, 49), generator=g)
    ref = th * lv * tilt
    pert = 10 ** ((torch.rand((batch, frames, 49), generator=g) - 0.5) * 2 * spread)
    return ref.float().contiguous(), (ref * pert).float().contiguous()


def _chain_errors(chain, ref, deg, seed):
    """Relative errors of the chain's outputs and gradients against float64."""

    batch = ref.shape[0]
    g = torch.Generator().manual_seed(seed + 1)
    up = [torch.randn(batch, generator=g, dtype=torch.float64) for _ in range(2)]
    r, d = ref.cuda().requires_grad_(True), deg.cuda().requires_grad_(True)
    ds, da = chain(r, d)
    gr, gd = torch.autograd.grad([ds, da], [r, d], grad_outputs=[u.float().cuda() for u in up])
    ro, do = ref.double().requires_grad_(True), deg.double().requires_grad_(True)
    wds, wda = O.chain(ro, do)
    wr, wd = torch.autograd.grad([wds, wda], [ro, do], grad_outputs=up)
    errs = {}
    for name, got, want in (("symm", ds, wds), ("asymm", da, wda), ("gref", gr, wr), ("gdeg", gd, wd)):
        got = got.detach().double().cpu()
        assert torch.isfinite(got).all(), name
        diff = float((got - want.detach()).abs().max())
        scale = float(want.detach().abs().max())
        errs[name] = diff / scale if scale > 0 else diff
    return errs


def _check(errs, what):
    for name in ("symm", "asymm"):
        assert errs[name] <= CHAIN_FWD, (what, name, errs)
    for name in ("gref", "gdeg"):
        assert errs[name] <= CHAIN_GRAD, (what, name, errs)


def test_chain_random_fuzz(chain):
    """The reference's 60 point sweep: batch 1..8, 20..260 frames, spreads of
    0.05 to 4 decades, levels over 1 to 9 decades."""

    rng = random.Random(0)
    worst = dict.fromkeys(("symm", "asymm", "gref", "gdeg"), 0.0)
    for i in range(60):
        batch = rng.choice([1, 1, 2, 3, 5, 8])
        frames = rng.randint(20, 260)
        spread = rng.choice([0.05, 0.2, 0.5, 1.0, 2.0, 4.0])
        level = rng.choice([1.0, 3.0, 6.0, 9.0])
        ref, deg = _spectra(batch, frames, seed=i * 977 + 3, spread=spread, level=level)
        errs = _chain_errors(chain, ref, deg, seed=i)
        _check(errs, (i, batch, frames, spread, level))
        for name, value in errs.items():
            worst[name] = max(worst[name], value)
    print("\nchain fuzz worst " + " ".join(f"{k}={v:.2e}" for k, v in worst.items()))


@pytest.mark.parametrize("factor", [1e-6, 1e6])
def test_chain_ratio_clamp_branches(chain, factor):
    """``test_triton_chain.py:332-362``: deg = 1e-6 ref drives the band ratio to
    its 0.01 clamp, deg = 1e6 ref the frame ratio to its 3e-4 clamp."""

    ref, _ = _spectra(3, 63, seed=101)
    deg = (ref * factor).contiguous()
    th = O.constants()["threshs"].float()
    silent = (ref * (ref > th * 1e2)).sum(dim=2) < 1e7
    mask_ref = (ref > th * 100.0) * (~silent.unsqueeze(2))
    mask_deg = (deg > th * 100.0) * (~silent.unsqueeze(2))
    ratio = ((deg * mask_deg).mean(dim=1) + 1000) / ((ref * mask_ref).mean(dim=1) + 1000)
    equ_ref = ratio.unsqueeze(1).clamp(0.01, 100.0) * ref
    taer = (equ_ref * (equ_ref > th)).sum(dim=2)
    fpr = (taer + 5e3) / ((deg * (deg > th)).sum(dim=2) + 5e3)
    if factor < 1.0:
        assert (ratio < 0.01).any()
    else:
        assert (fpr < 3e-4).any()
    _check(_chain_errors(chain, ref, deg, seed=2), factor)


def _single_band(k, ref_level, deg_level, frames=40):
    ref = torch.zeros(1, frames, 49)
    deg = torch.zeros(1, frames, 49)
    ref[:, :, k] = ref_level
    deg[:, :, k] = deg_level
    return ref.contiguous(), deg.contiguous()


def _clamp_case(case):
    """Inputs of the oracle's clamp known answers (``test_oracle.py``)."""

    th = O.constants()["threshs"]
    a = 2e7
    return {
        "45 cap": (40, a, 1e7 * a),
        "band ratio 0.01, asymmetry cut": (25, a, 1e-6 * a),
        "band ratio 100, frame ratio 3e-4": (10, a, 1.5e6 * a),
        "asymmetry cap 12": (10, a, 3e6 * a),
        "frame ratio 5": (25, a, float(th[25]) / 6),
        "frame ratio 5, audible": (25, a, float(th[25]) / 3),
    }[case]


@pytest.mark.parametrize(
    "case",
    ["45 cap", "band ratio 0.01, asymmetry cut", "band ratio 100, frame ratio 3e-4",
     "asymmetry cap 12", "frame ratio 5", "frame ratio 5, audible"],
)
def test_chain_clamp_known_answer_inputs(chain, case):
    ref, deg = _single_band(*_clamp_case(case))
    _check(_chain_errors(chain, ref, deg, seed=3), case)


@pytest.mark.parametrize("deg_scale", [1.0, 100.0])
def test_chain_exact_threshold_values(chain, deg_scale):
    """``test_triton_chain.py:725-750``: spectra at the float32 hearing thresholds.

    The chain compares the float32 spectra with the float64 thresholds, as
    upstream ``PesqLoss`` does (its threshold buffer is float64), so the bands
    whose float32 threshold rounds up are just audible; the result is the
    oracle's on the same values, not the 1e-20 floor of the exact-threshold
    known answer (``test_oracle.py``), which needs float64 spectra.
    """

    th = chain.threshs.detach().cpu().reshape(1, 1, -1)
    ref = th.expand(2, 62, 49).contiguous()
    deg = (th * deg_scale).expand(2, 62, 49).contiguous()
    errs = _chain_errors(chain, ref, deg, seed=4)
    _check(errs, deg_scale)
    ds, da = chain(ref.cuda(), deg.cuda())
    assert math.isfinite(float(ds.sum())) and math.isfinite(float(da.sum()))


# -- chain: the rest of the reference's chain contract ------------------------------


def _grad_pair(chain, ref, deg, weights, oracle=False):
    """Gradients of ``sum(w0 d_symm + w1 d_asymm)`` w.r.t. both spectra."""

    if oracle:
        r, d = ref.double().requires_grad_(True), deg.double().requires_grad_(True)
        ds, da = O.chain(r, d)
        w = [x.double() for x in weights]
    else:
        r, d = ref.cuda().requires_grad_(True), deg.cuda().requires_grad_(True)
        ds, da = chain(r, d)
        w = [x.float().cuda() for x in weights]
    total = (ds * w[0]).sum() + (da * w[1]).sum()
    grads = torch.autograd.grad(total, [r, d])
    return [g.detach().double().cpu() for g in grads]


@pytest.mark.parametrize("u", [1e-2, 1e-3])
def test_chain_near_threshold_bands(chain, u):
    """``test_triton_chain.py:455-495``: every band a relative ``u`` above its
    hearing threshold, where ``(0.5 + 0.5 x / th)^e - 1`` cancels to the last
    digits unless the loudness is formed as ``expm1(e log1p(.))``.  The
    reference's float32 chain is held to 1e-5 / 5e-5 (u = 1e-2) and
    1.2e-4 / 6e-4 (u = 1e-3) there; the kernels here keep the chain in float64
    and are held to the fuzz budgets of this file (1e-6 forward, 1e-5
    gradients), which the reference's float32 spelling would fail."""

    th = O.constants()["threshs"].float().reshape(1, 1, -1)
    g = torch.Generator().manual_seed(7)
    shape = (3, 63, 49)
    ref = th * (1.0 + u * (0.5 + torch.rand(shape, generator=g)))
    deg = th * (1.0 + u * (0.5 + torch.rand(shape, generator=g)))
    # every band is audible: the loudness of every (frame, band) is formed
    assert bool((ref.double() > th.double()).all()) and bool((deg.double() > th.double()).all())
    errs = _chain_errors(chain, ref.contiguous(), deg.contiguous(), seed=1)
    print(f"\nnear threshold u={u:g}: " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()))
    _check(errs, u)


def test_chain_many_silent_frames(chain):
    """``test_triton_chain.py:314-329``: most frames below the 1e7 total audible
    energy of the silence test (they drop out of the band means)."""

    ref, deg = _spectra(4, 71, seed=11)
    g = torch.Generator().manual_seed(12)
    silent = torch.rand((4, 71, 1), generator=g) < 0.8
    ref = torch.where(silent, ref * 1e-7, ref).contiguous()
    deg = torch.where(silent, deg * 1e-7, deg).contiguous()
    th = O.constants()["threshs"]
    is_silent = (ref.double() * (ref.double() > th * 1e2)).sum(dim=2) < 1e7
    assert 0.5 < is_silent.double().mean().item() < 1.0
    _check(_chain_errors(chain, ref, deg, seed=13), "silent")


def test_chain_frames_outside_windows(chain):
    """``test_triton_chain.py:774-796``: with 29 frames there is one window
    (frames 0..19); frames 20..28 reach the distances only through the band
    means, and their gradient is that path's, non-zero, and the oracle's."""

    ref, deg = _spectra(2, 29, seed=61)
    weights = [torch.ones(2, dtype=torch.float64)] * 2
    got = _grad_pair(chain, ref, deg, weights)
    want = _grad_pair(chain, ref, deg, weights, oracle=True)
    scale = max(float(w.abs().max()) for w in want)
    for mine, oracle in zip(got, want):
        assert torch.isfinite(mine).all()
        assert float((mine[:, 20:] - oracle[:, 20:]).abs().max()) <= CHAIN_GRAD * scale
        assert float((mine - oracle).abs().max()) <= CHAIN_GRAD * scale
        assert float(mine[:, 20:].abs().max()) > 0.0


@pytest.mark.parametrize("which", [0, 1])
def test_chain_single_output_gradient(chain, which):
    """``test_triton_chain.py:405-425``: only d_symm (or only d_asymm) carries
    an upstream gradient; the other output's backward is absent, not zero."""

    ref, deg = _spectra(2, 62, seed=109)
    up = torch.randn(2, generator=torch.Generator().manual_seed(4), dtype=torch.float64)
    r, d = ref.cuda().requires_grad_(True), deg.cuda().requires_grad_(True)
    out = chain(r, d)[which]
    got = torch.autograd.grad((out * up.float().cuda()).sum(), [r, d])
    ro, do = ref.double().requires_grad_(True), deg.double().requires_grad_(True)
    want = torch.autograd.grad((O.chain(ro, do)[which] * up).sum(), [ro, do])
    scale = max(float(w.abs().max()) for w in want)
    for mine, oracle in zip(got, want):
        mine = mine.double().cpu()
        assert torch.isfinite(mine).all()
        assert float((mine - oracle).abs().max()) <= CHAIN_GRAD * scale


def test_chain_aliased_inputs(chain):
    """``test_triton_chain.py:386-403``: one tensor passed as both spectra;
    autograd adds the two paths' gradients."""

    ref, _ = _spectra(2, 62, seed=401)
    both = ref.cuda().requires_grad_(True)
    ds, da = chain(both, both)
    (got,) = torch.autograd.grad(ds.sum() + da.sum(), both)
    both64 = ref.double().requires_grad_(True)
    wds, wda = O.chain(both64, both64)
    (want,) = torch.autograd.grad(wds.sum() + wda.sum(), both64)
    got = got.double().cpu()
    assert torch.isfinite(got).all()
    assert float((got - want).abs().max()) <= CHAIN_GRAD * float(want.abs().max())
    ds, wds = ds.detach().double().cpu(), wds.detach()
    assert float((ds - wds).abs().max()) <= CHAIN_FWD * float(wds.abs().max())


def test_chain_empty_batch(chain):
    """``test_triton_chain.py:799-806``: a zero sized batch is a no-op that
    returns empty distances (and an empty gradient), not a launch failure."""

    empty = torch.zeros(0, 62, 49, device="cuda", requires_grad=True)
    ds, da = chain(empty, empty)
    assert ds.shape == (0,) and da.shape == (0,)
    (g,) = torch.autograd.grad(ds.sum() + da.sum(), empty)
    assert g.shape == empty.shape


@pytest.mark.parametrize("rate,samples", [(16000, 24000), (48000, 72000)])
def test_loss_empty_batch(model, rate, samples):
    """The whole loss of an empty batch: empty outputs and gradients."""

    m = model if rate == 16000 else PesqLossTriton(0.5, sample_rate=rate).cuda()
    r = torch.zeros(0, samples, device="cuda")
    d = torch.zeros(0, samples, device="cuda", requires_grad=True)
    loss = m(r, d)
    assert loss.shape == (0,)
    (g,) = torch.autograd.grad(loss.sum(), d)
    assert g.shape == d.shape
    assert m.mos(r, d.detach()).shape == (0,)
    ds, da = m.raw(r, d.detach())
    assert ds.shape == (0,) and da.shape == (0,)
