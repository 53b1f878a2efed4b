"""GPU parity of the stand-alone stage operators against the float64 oracle.

Mirrors ``test_triton_elementwise.py``, ``test_triton_spectral.py`` and
``test_triton_chain.py`` of the reference.  Tolerances:

* ``peak_normalize`` and ``edge_ramp``: bit exact with float32 PyTorch (the
  reference's own claim, ``test_triton_elementwise.py:1-16``);
* ``align_scale`` / ``pesq_epilogue``: 1e-6 relative to float64 closed forms
  (float64 reductions inside);
* ``HipStftBark``: ``|got - want| <= 1e-6 |want| + 1e-6 * frame peak`` forward
  (reference budget: 1e-5 and 5e-6), backward ``1e-5`` of the sample scale;
* ``HipPesqChain``: the kernels evaluate the chain in float64 on the same
  float32 spectra as the oracle; what remains is the float32 rounding of the
  outputs (6e-8), so forward and gradients 3e-7 relative (reference budgets
  6e-6 / 3e-5).
"""

import numpy as np
import pytest
import torch

from oracle import pesq_oracle as O
from torch_pesq import PesqLoss
from torch_pesq.hip_ops.chain import HipPesqChain
from torch_pesq.hip_ops.elementwise import align_scale, edge_ramp, peak_normalize, pesq_epilogue
from torch_pesq.hip_ops.spectral import HipStftBark

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model():
    return PesqLoss(1.0, sample_rate=16000).cuda()


# -- peak normalisation -------------------------------------------------------


@pytest.mark.parametrize("stack", [False, True])
def test_peak_normalize_bit_exact(stack):
    g = torch.Generator(device="cuda").manual_seed(0)
    ref = torch.randn(3, 20001, device="cuda", generator=g) * 3
    deg = torch.randn(3, 20001, device="cuda", generator=g)
    peak = torch.max(ref.abs().amax(1, keepdim=True), deg.abs().amax(1, keepdim=True))
    out = peak_normalize(ref, deg, stack=stack)
    if stack:
        assert out.shape == (6, 20001)
        out = (out[:3], out[3:])
    assert torch.equal(out[0], ref / peak) and torch.equal(out[1], deg / peak)


def test_peak_normalize_backward_treats_peak_as_constant():
    ref = torch.randn(2, 1000, device="cuda", requires_grad=True)
    deg = torch.randn(2, 1000, device="cuda", requires_grad=True)
    stacked = peak_normalize(ref, deg, stack=True)
    g = torch.randn_like(stacked)
    g_ref, g_deg = torch.autograd.grad(stacked, [ref, deg], grad_outputs=g)
    peak = torch.max(ref.abs().amax(1, keepdim=True), deg.abs().amax(1, keepdim=True)).detach()
    assert torch.equal(g_ref, g[:2] / peak) and torch.equal(g_deg, g[2:] / peak)
    # only the degraded input requires a gradient
    ref2 = ref.detach()
    (g_deg_only,) = torch.autograd.grad(peak_normalize(ref2, deg, stack=True), [deg], grad_outputs=g)
    assert torch.equal(g_deg_only, g_deg)


def test_peak_normalize_errors():
    with pytest.raises(RuntimeError):
        peak_normalize(torch.randn(2, 10, device="cuda"), torch.randn(2, 11, device="cuda"))
    with pytest.raises(RuntimeError):
        peak_normalize(torch.randn(2, 0, device="cuda"), torch.randn(2, 0, device="cuda"))
    with pytest.raises(RuntimeError):
        peak_normalize(torch.randn(2, 10), torch.randn(2, 10))


# -- edge ramp ----------------------------------------------------------------


@pytest.mark.parametrize("n", [15, 16, 29, 30, 31, 1000])
def test_edge_ramp_bit_exact(n):
    x = torch.randn(3, n, device="cuda")
    emp = torch.linspace(0, 15, 16, device="cuda")[1:] / 16.0
    want = x.clone()
    want[:, :15] *= emp
    want[:, -15:] *= torch.flip(emp, dims=(0,))
    assert torch.equal(edge_ramp(x), want)
    xg = x.clone().requires_grad_(True)
    g = torch.randn_like(x)
    (gx,) = torch.autograd.grad(edge_ramp(xg), xg, grad_outputs=g)
    assert torch.equal(gx, edge_ramp(g))


def test_edge_ramp_needs_15_samples():
    with pytest.raises(RuntimeError):
        edge_ramp(torch.randn(2, 14, device="cuda"))


# -- level alignment ----------------------------------------------------------


def test_align_scale_matches_float64():
    g = torch.Generator().manual_seed(1)
    signal = torch.randn(3, 9000, generator=g, dtype=torch.float64)
    filtered = torch.randn(3, 9000, generator=g, dtype=torch.float64) * 0.3
    s, f = signal.float().cuda().requires_grad_(True), filtered.float().cuda().requires_grad_(True)
    out = align_scale(s, f)
    so, fo = s.detach().double().cpu().requires_grad_(True), f.detach().double().cpu().requires_grad_(True)
    power = (fo**2).sum(1, keepdim=True) / (9000 + 5120) / 1.04684
    want = so * (1e7 / power).sqrt()
    assert float(((out.double().cpu() - want).abs() / want.abs().max()).max()) < 1e-6
    w = torch.randn(3, 9000, generator=g, dtype=torch.float64)
    gs, gf = torch.autograd.grad(out, [s, f], grad_outputs=w.float().cuda())
    ws, wf = torch.autograd.grad(want, [so, fo], grad_outputs=w)
    assert float((gs.double().cpu() - ws).abs().max() / ws.abs().max()) < 1e-6
    assert float((gf.double().cpu() - wf).abs().max() / wf.abs().max()) < 1e-6


def test_align_level_and_preemphasize_match_oracle(model):
    x = torch.randn(2, 12000, dtype=torch.float64, generator=torch.Generator().manual_seed(2)) * 0.1
    got = model.align_level(x.float().cuda())
    want = O.align_level(x.float().double())
    assert float((got.double().cpu() - want).abs().max() / want.abs().max()) < 1e-6
    got = model.preemphasize(x.float().cuda())
    want = O.preemphasize(x.float().double())
    assert float((got.double().cpu() - want).abs().max() / want.abs().max()) < 1e-6


# -- epilogue -----------------------------------------------------------------


def test_epilogue_matches_closed_form():
    ds = torch.tensor([0.0, 5.0, 20.0, 44.0], device="cuda", requires_grad=True)
    da = torch.tensor([0.0, 10.0, 30.0, 45.0], device="cuda", requires_grad=True)
    mos, loss = pesq_epilogue(ds, da, 0.5)
    dso, dao = ds.detach().double().cpu().requires_grad_(True), da.detach().double().cpu().requires_grad_(True)
    wmos, wloss = O.epilogue(dso, dao, 0.5)
    assert float(((mos.double().cpu() - wmos).abs() / wmos).max()) < 1e-6
    assert float(((loss.double().cpu() - wloss).abs() / wloss.clamp(min=1e-30)).max()) < 1e-6
    for outs, wouts in (((mos,), (wmos,)), ((loss,), (wloss,)), ((mos, loss), (wmos, wloss))):
        gw = [torch.full_like(o, 0.7) for o in outs]
        got = torch.autograd.grad(outs, [ds, da], grad_outputs=gw, retain_graph=True)
        want = torch.autograd.grad(wouts, [dso, dao], grad_outputs=[g.double().cpu() for g in gw], retain_graph=True)
        for gg, ww in zip(got, want):
            assert float((gg.double().cpu() - ww).abs().max() / ww.abs().max()) < 1e-6
    with pytest.raises(RuntimeError):
        pesq_epilogue(ds, da, torch.tensor(1.0, requires_grad=True))


# -- STFT / Bark ----------------------------------------------------------------


@pytest.fixture(scope="module")
def stft(model):
    return HipStftBark(model.to_spec.window, model.fbank.fbank, model.fbank.pow_dens_correction).cuda()


def _frame_close(got, want, rtol=1e-6, atol_scale=1e-6):
    got = got.double().cpu()
    scale = want.abs().amax(2, keepdim=True)
    return bool(((got - want).abs() <= rtol * want.abs() + atol_scale * scale).all())


@pytest.mark.parametrize("n,n_padded", [(4000, None), (4000, 4096), (3900, 4096), (20000, 20032), (777, 1024)])
def test_stft_bark_forward(stft, n, n_padded):
    x = torch.randn(3, n, generator=torch.Generator().manual_seed(n)) * 1000.0
    got = stft(x.cuda(), n_padded)
    padded = n if n_padded is None else n_padded
    xp = torch.nn.functional.pad(x.double(), (0, padded - n))
    # oracle: frames over the given padded length (no extra N % 256 padding here)
    c = O.constants()
    spec = torch.stft(xp, 512, 256, 512, c["window"], center=False, return_complex=True).abs() ** 2
    spec = spec.swapaxes(1, 2)
    spec[:, :, 0] = 0
    want = torch.matmul(spec[:, :, :-1], c["fbank"].t()) * c["corr"]
    assert got.shape == want.shape == (3, 1 + (padded - 512) // 256, 49)
    assert _frame_close(got, want)


def test_stft_bark_drops_the_partial_frame(stft):
    x = torch.randn(2, 4000, device="cuda") * 1000.0
    out = stft(x)
    assert out.shape[1] == 14
    tail = x.clone()
    tail[:, 3840:] = 1e9
    assert torch.equal(stft(tail), out)


def test_stft_bark_backward(stft):
    x = (torch.randn(2, 6000, generator=torch.Generator().manual_seed(3)) * 100.0)
    xg = x.cuda().requires_grad_(True)
    out = stft(xg)
    w = torch.randn(out.shape, generator=torch.Generator().manual_seed(4), dtype=torch.float64)
    (got,) = torch.autograd.grad(out, xg, grad_outputs=w.float().cuda())
    xo = x.double().requires_grad_(True)
    c = O.constants()
    spec = torch.stft(xo, 512, 256, 512, c["window"], center=False, return_complex=True).abs() ** 2
    spec = spec.swapaxes(1, 2)
    spec = torch.cat([torch.zeros_like(spec[:, :, :1]), spec[:, :, 1:]], 2)
    want_out = torch.matmul(spec[:, :, :-1], c["fbank"].t()) * c["corr"]
    (want,) = torch.autograd.grad(want_out, xo, grad_outputs=w)
    assert float((got.double().cpu() - want).abs().max() / want.abs().max()) < 1e-5
    # samples behind the last frame get no gradient
    frames = out.shape[1]
    assert torch.count_nonzero(got[:, 256 * (frames + 1) :]) == 0


def test_stft_bark_errors(stft):
    with pytest.raises(ValueError):
        stft(torch.randn(2, 1000, device="cuda"), 900)
    with pytest.raises(ValueError):
        stft(torch.randn(2, 300, device="cuda"))
    with pytest.raises(ValueError):
        HipStftBark(torch.hann_window(512), torch.eye(49, 256), torch.ones(49), n_fft=256)


# -- perceptual chain ------------------------------------------------------------


@pytest.fixture(scope="module")
def chain(model):
    return HipPesqChain(model.loudness.threshs, model.loudness.exp, model.fbank.width_bark,
                        model.fbank.total_width).cuda()


def _spectra(batch, frames, seed, spread=0.5, level=6.0):
    """Log-uniform spectra straddling the thresholds (``test_triton_chain.py:95-113``)."""

    g = torch.Generator().manual_seed(seed)
    th = O.constants()["threshs"].float()
    lv = 10 ** (torch.rand((batch, frames, 1), generator=g) * level)
    tilt = 0.2 + 2.0 * torch.rand((batch, frames, 49), generator=g)
    ref = th * lv * tilt
    pert = 10 ** ((torch.rand((batch, frames, 49), generator=g) - 0.5) * 2 * spread)
    return ref.float().contiguous(), (ref * pert).float().contiguous()


@pytest.mark.parametrize("batch,frames,seed,spread", [(1, 20, 0, 0.5), (3, 57, 1, 0.5), (2, 260, 2, 2.0), (4, 499, 3, 0.05)])
def test_chain_forward_and_gradients(chain, batch, frames, seed, spread):
    ref, deg = _spectra(batch, frames, seed, spread)
    r, d = ref.cuda().requires_grad_(True), deg.cuda().requires_grad_(True)
    ds, da = chain(r, d)
    ro, do = ref.double().requires_grad_(True), deg.double().requires_grad_(True)
    wds, wda = O.chain(ro, do)
    assert float(((ds.double().cpu() - wds).abs() / wds).max()) < 3e-7
    assert float(((da.double().cpu() - wda).abs() / wda).max()) < 3e-7
    u = torch.randn(batch, dtype=torch.float64, generator=torch.Generator().manual_seed(seed + 10))
    v = torch.randn(batch, dtype=torch.float64, generator=torch.Generator().manual_seed(seed + 11))
    gr, gd = torch.autograd.grad([ds, da], [r, d], grad_outputs=[u.float().cuda(), v.float().cuda()])
    wr, wd = torch.autograd.grad([wds, wda], [ro, do], grad_outputs=[u, v])
    assert float((gr.double().cpu() - wr).abs().max() / wr.abs().max()) < 3e-7
    assert float((gd.double().cpu() - wd).abs().max() / wd.abs().max()) < 3e-7


def test_chain_identical_inputs(chain):
    ref, _ = _spectra(2, 40, 5)
    ds, da = chain(ref.cuda(), ref.cuda())
    assert torch.all(ds < 1e-19) and torch.all(da < 1e-19)


def test_chain_batch_independence_and_errors(chain):
    ref, deg = _spectra(3, 30, 6)
    ds, da = chain(ref.cuda(), deg.cuda())
    ds1, da1 = chain(ref[1:2].cuda(), deg[1:2].cuda())
    assert torch.equal(ds[1:2], ds1) and torch.equal(da[1:2], da1)
    with pytest.raises(ValueError):
        chain(ref[:, :19].cuda(), deg[:, :19].cuda())
    with pytest.raises(ValueError):
        chain(ref.cuda(), deg[:, :29].cuda())
    with pytest.raises(RuntimeError):
        chain(ref, deg)


@pytest.mark.parametrize("batch,frames", [(8, 63), (8, 1100)])
def test_chain_batch_independence_with_gradients(chain, batch, frames):
    """Every row of a batched call, outputs and both input gradients under
    per-row upstream gradients, equals the same row computed on its own, bit
    for bit (``test_triton_chain.py:568-598``, whose shape is the first case).
    In the second the batch (552 chain tiles) runs the wide kernel variants
    (four frames per wavefront) and each row alone (69 tiles) the narrow
    ones."""

    ref, deg = _spectra(batch, frames, 999)
    g = torch.Generator().manual_seed(5)
    up_s = torch.randn(batch, generator=g).cuda()
    up_a = torch.randn(batch, generator=g).cuda()
    r, d = ref.cuda().requires_grad_(True), deg.cuda().requires_grad_(True)
    symm, asymm = chain(r, d)
    grads = torch.autograd.grad((symm * up_s).sum() + (asymm * up_a).sum(), (r, d))
    for b in range(batch):
        rb = ref[b : b + 1].cuda().requires_grad_(True)
        db = deg[b : b + 1].cuda().requires_grad_(True)
        symm_b, asymm_b = chain(rb, db)
        grads_b = torch.autograd.grad(
            (symm_b * up_s[b : b + 1]).sum() + (asymm_b * up_a[b : b + 1]).sum(), (rb, db)
        )
        assert torch.equal(symm[b : b + 1], symm_b), b
        assert torch.equal(asymm[b : b + 1], asymm_b), b
        assert torch.equal(grads[0][b : b + 1], grads_b[0]), b
        assert torch.equal(grads[1][b : b + 1], grads_b[1]), b


@pytest.mark.parametrize("nband", [17, 33, 64, 65, 100, 128])
def test_chain_other_band_counts(nband):
    """Band counts other than 49 (``test_triton_chain.py:668-717``): random
    thresholds, exponents and widths, against the float64 restatement with the
    same tables, forward and gradients.  The kernels take one band per lane up
    to 64 bands and two (band lane + 64) up to 128, the largest count (129
    raises)."""

    gen = torch.Generator().manual_seed(nband)
    threshs = (10 ** (torch.rand(nband, generator=gen) * 8 - 1)).double()
    exps = (0.15 + 0.15 * torch.rand(nband, generator=gen)).double()
    widths = (0.15 + 0.45 * torch.rand(nband, generator=gen)).double()
    total = float(widths[1:].sum())
    chain = HipPesqChain(threshs, exps, widths, total, 0.1866055).cuda()
    level = 10 ** (torch.rand((2, 63, 1), generator=gen, dtype=torch.float64) * 6)
    tilt = 0.2 + 2.0 * torch.rand((2, 63, nband), generator=gen, dtype=torch.float64)
    ref = (threshs.reshape(1, 1, -1) * level * tilt).float()
    deg = (ref.double() * 10 ** (torch.rand((2, 63, nband), generator=gen, dtype=torch.float64) - 0.5)).float()
    c = dict(O.constants())
    c.update(threshs=threshs, exp=exps, width_bark=widths, total_width=torch.tensor(total, dtype=torch.float64))
    r, d = ref.cuda().requires_grad_(True), deg.cuda().requires_grad_(True)
    ds, da = chain(r, d)
    ro, do = ref.double().requires_grad_(True), deg.double().requires_grad_(True)
    wds, wda = O.chain(ro, do, c)
    assert float(((ds.double().cpu() - wds).abs() / wds).max()) < 1e-5
    assert float(((da.double().cpu() - wda).abs() / wda).max()) < 1e-5
    u = torch.tensor([0.7, -1.3], dtype=torch.float64)
    gr, gd = torch.autograd.grad([ds.sum(), (da * u.float().cuda()).sum()], [r, d])
    wr, wd = torch.autograd.grad([wds.sum(), (wda * u).sum()], [ro, do])
    assert float((gr.double().cpu() - wr).abs().max() / wr.abs().max()) < 2e-5
    assert float((gd.double().cpu() - wd).abs().max() / wd.abs().max()) < 2e-5
    with pytest.raises(ValueError, match="Bark bands"):
        chain(ref[:, :, :-1].contiguous().cuda(), deg[:, :, :-1].contiguous().cuda())


def test_chain_rejects_more_than_128_bands():
    with pytest.raises(ValueError, match="at most 128"):
        HipPesqChain(torch.ones(129), torch.full((129,), 0.2), torch.ones(129), 128.0)
