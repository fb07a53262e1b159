"""Flow-matching Euler sampler (kiln_amd.sampler; the reference's sample() for sampler "euler", scheduler
"simple", engine/src/pipeline.cu:66-78, 304-331, 415-552)."""
import numpy as np
import pytest
import torch

import kiln_amd
from kiln_amd import sampler

DEV = "cuda:0"


def test_flow_sigmas_closed_forms():
    # shift 1: the linear ramp 1 .. 1/steps, then 0
    np.testing.assert_allclose(sampler.flow_sigmas(4, 1.0), [1.0, 0.75, 0.5, 0.25, 0.0], rtol=0, atol=1e-7)
    # shift 3: t' = 3t / (1 + 2t) at t = 1, 7/8, ..., 1/8
    t = np.arange(8, 0, -1) / 8.0
    np.testing.assert_allclose(sampler.flow_sigmas(8, 3.0)[:-1], 3 * t / (1 + 2 * t), rtol=1e-6)
    # partial denoise: the last steps + 1 sigmas of the schedule of steps / denoise
    np.testing.assert_allclose(sampler.flow_sigmas(4, 1.0, 0.5), [0.5, 0.375, 0.25, 0.125, 0.0], rtol=0, atol=1e-7)


@pytest.mark.gpu
def test_flow_kernels_and_euler_cfg_loop(gpu):
    """flow_start / flow_euler_step against numpy in the reference's arithmetic, then a 4-step CFG sampling loop
    with a stub velocity model (v = 0.5 x + c for the prompt, 0.25 x for the negative) against a numpy loop."""
    g = torch.Generator().manual_seed(3)
    x0, noise, init = (torch.randn(16, 6, 10, generator=g) for _ in range(3))
    x = torch.empty(16, 6, 10, device=DEV)
    kiln_amd.flow_start(x, noise.to(DEV), 0.8, init.to(DEV))
    np.testing.assert_allclose(x.cpu().numpy(), (np.float32(0.8) * noise.numpy() + np.float32(0.2) * init.numpy()),
                               rtol=1e-6, atol=1e-6)
    v = torch.randn(16, 6, 10, generator=g)
    xd = x0.to(DEV)
    kiln_amd.flow_euler_step(xd, v.to(DEV), 0.8, 0.6)
    xn = x0.numpy()
    den = xn - v.numpy() * np.float32(0.8)
    np.testing.assert_allclose(xd.cpu().numpy(), xn + (xn - den) / np.float32(0.8) * np.float32(-0.2), rtol=1e-5,
                               atol=1e-6)

    c = torch.randn(16, 6, 10, generator=g)
    cd = c.to(DEV)
    calls = []

    def model(outs, xx, t, cfg_now):
        calls.append((round(t, 6), cfg_now))
        outs[0].copy_(0.5 * xx + cd)
        if cfg_now:
            outs[1].copy_(0.25 * xx)

    sig = sampler.flow_sigmas(4, 3.0)
    xg = torch.empty(16, 6, 10, device=DEV)
    sampler.sample_euler(model, xg, noise.to(DEV), sig, cfg=4.0, cfg_until=0.5, timestep_mult=1000.0)
    xr = sig[0] * noise.numpy().astype(np.float64)
    for i in range(4):
        vp = 0.5 * xr + c.numpy()
        if i < 2:
            vp = 0.25 * xr + 4.0 * (vp - 0.25 * xr)
        xr = xr + vp * (sig[i + 1] - sig[i])
    # the model's timestep is float32 sigma * timestep_mult (pipeline.cu:484)
    assert calls == [(round(float(np.float32(s) * np.float32(1000.0)), 6), i < 2) for i, s in enumerate(sig[:-1])]
    np.testing.assert_allclose(xg.cpu().numpy(), xr, rtol=1e-4, atol=1e-4)


@pytest.mark.gpu
def test_step_cache_guards(gpu):
    """The sampler's cache guards (engine/src/pipeline.cu:463-480): no skip before max(2, ceil(0.15 steps)), none
    in the last max(1, ceil(0.1 steps)) steps, at most cache_max_hits in a row. A stub model records `allow` and
    skips whenever allowed."""
    class Cache:  # a stand-in with the attributes the sampler reads and sets
        def __init__(self, threshold):
            self.threshold, self.allow, self.skipped, self.skips = threshold, False, False, 0

    class Stub:
        def __init__(self, cache):
            self.cache, self.allowed = cache, []

        def __call__(self, outs, xx, t, cfg_now):
            self.allowed.append(self.cache.allow)
            self.cache.skipped = self.cache.allow
            outs[0].zero_()

    sc = Cache(0.1)
    stub = Stub(sc)
    x = torch.empty(16, 4, 4, device=DEV)
    sampler.sample_euler(stub, x, torch.zeros(16, 4, 4, device=DEV), sampler.flow_sigmas(20, 3.0), negative=False,
                         cache=sc)
    # steps 0-2 warm (ceil(0.15 * 20) = 3), last 2 (ceil(0.1 * 20)) off, then 2 skips and one full step repeating
    expect = [False] * 3 + [True, True, False] * 5
    expect = (expect + [False] * 20)[:18] + [False, False]
    assert stub.allowed == expect and sc.skips == sum(expect)


@pytest.mark.parametrize("name", ["euler", "dpmpp_2m", "res_multistep"])
def test_step_coef_exact_on_linear_trajectories(name):
    """Every step x <- a x + b den + c old (engine/src/pipeline.cu:396-411) must keep a point of a straight flow
    trajectory x(s) = x0 + s (n - x0) on it when den = old = x0: a = s'/s and b + c = 1 - s'/s (to float32, the
    coefficients' type in the reference)."""
    sig = sampler.flow_sigmas(10, 3.0)
    for i in range(10):
        a, b, c = sampler.step_coef(name, sig, i, i > 0)
        sn, s = sig[i + 1], sig[i]
        assert abs(a - sn / s) < 1e-6 and abs(b + c - (1 - sn / s)) < 1e-6
    # first step and the step to sigma 0 are first order
    assert sampler.step_coef(name, sig, 0, False)[2] == 0.0 and sampler.step_coef(name, sig, 9, True)[2] == 0.0


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["euler", "dpmpp_2m", "res_multistep", "euler_ancestral"])
def test_samplers_on_a_straight_trajectory(gpu, name):
    """A model with constant velocity v = n - x0 (a straight trajectory from the noise n to x0): the
    deterministic samplers land on x0; the ancestral one against a float64 statement of its step with the
    library's torch_randn noise."""
    g = torch.Generator().manual_seed(11)
    x0, n = torch.randn(16, 4, 6, generator=g), torch.randn(16, 4, 6, generator=g)
    vd = (n - x0).to(DEV)

    def model(outs, xx, t, cfg_now):
        outs[0].copy_(vd)

    sig = sampler.flow_sigmas(6, 3.0)
    x = torch.empty(16, 4, 6, device=DEV)
    sampler.sample_euler(model, x, n.to(DEV), sig, negative=False, sampler=name, seed=5)
    if name != "euler_ancestral":
        np.testing.assert_allclose(x.cpu().numpy(), x0.numpy(), rtol=0, atol=2e-5)
        return
    xr, v = sig[0] * n.double(), (n - x0).double()
    for i in range(6):
        s, sn = sig[i], sig[i + 1]
        den = xr - v * s
        if sn == 0.0:
            xr = den
            continue
        sd = sn * (1.0 + (sn / s - 1.0))
        aip1, ad = 1.0 - sn, 1.0 - sd
        renoise = max(0.0, sn * sn - sd * sd * aip1 * aip1 / (ad * ad)) ** 0.5
        r, a = sd / s, aip1 / ad
        xr = a * r * xr + a * (1 - r) * den + renoise * kiln_amd.torch_randn(5 + 1 + i, xr.numel()).view_as(xr).double()
    np.testing.assert_allclose(x.cpu().double().numpy(), xr.numpy(), rtol=0, atol=2e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["euler", "dpmpp_2m"])
def test_inpainting_mask(gpu, name):
    """Inpainting (engine/src/pipeline.cu:309-324): mask 1 everywhere samples as without a mask; mask 0 everywhere
    returns the init exactly at sigma 0; a half mask keeps the init outside and matches the unmasked result
    inside for a model that does not mix pixels (v = x - init, per pixel)."""
    g = torch.Generator().manual_seed(12)
    init, n = torch.randn(16, 4, 6, generator=g).to(DEV), torch.randn(16, 4, 6, generator=g).to(DEV)

    def model(outs, xx, t, cfg_now):
        outs[0].copy_(0.7 * xx - 0.3 * init)

    sig = sampler.flow_sigmas(5, 3.0, 0.8)
    ref = torch.empty_like(init)
    sampler.sample_euler(model, ref, n, sig, negative=False, init=init, sampler=name)
    x1 = torch.empty_like(init)
    sampler.sample_euler(model, x1, n, sig, negative=False, init=init, sampler=name, mask=torch.ones(4, 6, device=DEV))
    torch.testing.assert_close(x1, ref, rtol=1e-5, atol=1e-5)
    x0 = torch.empty_like(init)
    sampler.sample_euler(model, x0, n, sig, negative=False, init=init, sampler=name, mask=torch.zeros(4, 6, device=DEV))
    torch.testing.assert_close(x0, init, rtol=1e-5, atol=1e-5)
    m = torch.zeros(4, 6, device=DEV)
    m[:, :3] = 1
    xh = torch.empty_like(init)
    sampler.sample_euler(model, xh, n, sig, negative=False, init=init, sampler=name, mask=m)
    torch.testing.assert_close(xh[:, :, :3], ref[:, :, :3], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(xh[:, :, 3:], init[:, :, 3:], rtol=1e-5, atol=1e-5)


def test_schedulers_closed_forms():
    """Flow-space schedulers (engine/src/pipeline.cu:188-277): "simple" equals flow_sigmas; karras with rho 7 and
    exponential are geometric/power interpolations between sigma_max = 1 and sigma_min = shift(0.001) that end in
    0; kl_optimal is tan-linear in atan(sigma); every schedule is non-increasing and ends at 0; partial denoise
    takes the tail of the longer schedule."""
    import math
    for shift in (1.0, 3.0):
        np.testing.assert_allclose(sampler.schedule_sigmas("simple", 8, shift), sampler.flow_sigmas(8, shift), rtol=1e-7)
        smin = shift * 0.001 / (1 + (shift - 1) * 0.001)
        k = sampler.schedule_sigmas("karras", 5, shift)
        assert abs(k[0] - 1.0) < 1e-6 and abs(k[4] - smin) < 1e-6 and k[5] == 0.0
        r = [x ** (1 / 7) for x in k[:5]]
        np.testing.assert_allclose(np.diff(r), np.diff(r)[0], rtol=1e-4)
        e = sampler.schedule_sigmas("exponential", 5, shift)
        np.testing.assert_allclose(np.diff(np.log(e[:5])), math.log(smin) / 4, rtol=1e-5)
        kl = sampler.schedule_sigmas("kl_optimal", 5, shift)
        np.testing.assert_allclose(np.diff(np.arctan(kl[:5])), (math.atan(smin) - math.atan(1.0)) / 4, rtol=1e-5)
        for name in sampler.SCHEDULERS:
            s = sampler.schedule_sigmas(name, 10, shift)
            assert s[-1] == 0.0 and all(a >= b for a, b in zip(s, s[1:])), name
        full = sampler.schedule_sigmas("karras", 20, shift)
        np.testing.assert_allclose(sampler.schedule_sigmas("karras", 10, shift, 0.5), full[-11:], rtol=1e-7)


def test_ersde_coefficients_keep_the_data_point():
    """er_sde (engine/src/pipeline.cu:361-391) is exact for a sample that is all data: with x = (1 - s) x0 and
    den = x0 the noise-free part a x + b den equals (1 - s') x0, i.e. a (1 - s) + b = 1 - s'; the noise scale is
    real and non-negative; the stage grows 1, 2, 3."""
    sig = sampler.flow_sigmas(8, 3.0)
    sig[0] = 1.0 - 1e-4
    for i in range(7):
        a, b, c2, inv2, c3, inv3, cn, stage = sampler.ersde_coef(sig, i)
        assert abs(a * (1 - sig[i]) + b - (1 - sig[i + 1])) < 1e-6  # float32 coefficients, as the reference
        assert cn >= 0 and stage == min(3, i + 1)


@pytest.mark.gpu
def test_ersde_kernel_stages(gpu):
    """kiln_flow_ersde_step against a float64 statement of k_ersde for stages 1-3 (oldd written at stage >= 2)."""
    g = torch.Generator().manual_seed(13)
    x, den, old, oldd, nz = (torch.randn(1000, generator=g) for _ in range(5))
    for stage in (1, 2, 3):
        c = (0.7, 0.2, -0.3, -0.5, 0.1, -0.2, 0.4, stage)
        xd, od = x.to(DEV), oldd.to(DEV)
        kiln_amd.flow_ersde_step(xd, den.to(DEV), old.to(DEV), od, nz.to(DEV), c)
        v = 0.7 * x.double() + 0.2 * den.double()
        dd = (den.double() - old.double()) * -0.5
        if stage >= 2:
            v = v + -0.3 * dd
        if stage >= 3:
            v = v + 0.1 * (dd - oldd.double()) * -0.2
        v = v + 0.4 * nz.double()
        np.testing.assert_allclose(xd.cpu().double().numpy(), v.numpy(), rtol=1e-5, atol=1e-6)
        if stage >= 2:
            np.testing.assert_allclose(od.cpu().double().numpy(), dd.numpy(), rtol=1e-6, atol=1e-6)


@pytest.mark.gpu
def test_ersde_sampling_runs_deterministically(gpu):
    """A 6-step er_sde run (stages 1-3 and the final step to sigma 0) is finite and repeats bit for bit with the
    same seed (its noise is the library's torch_randn(seed + 1 + i))."""
    g = torch.Generator().manual_seed(14)
    x0, n = torch.randn(16, 4, 6, generator=g).to(DEV), torch.randn(16, 4, 6, generator=g).to(DEV)

    def model(outs, xx, t, cfg_now):
        outs[0].copy_(n - x0)

    sig = sampler.flow_sigmas(6, 3.0)
    runs = []
    for _ in range(2):
        x = torch.empty_like(x0)
        sampler.sample_euler(model, x, n, sig, negative=False, sampler="er_sde", seed=9)
        runs.append(x.cpu())
    assert torch.isfinite(runs[0]).all() and torch.equal(runs[0], runs[1])


def test_partial_denoise_uses_float32_denoise():
    """The reference computes total = (int)((double)steps / (double)denoise) with denoise a float
    (engine/src/pipeline.cu:67, 268): float32(0.8) = 0.800000011920929 makes 4 / 0.8 fall just below 5, so the
    schedule has 4 steps and steps 4 at denoise 0.8 is the full schedule from sigma 1."""
    np.testing.assert_allclose(sampler.flow_sigmas(4, 1.0, 0.8), [1.0, 0.75, 0.5, 0.25, 0.0], rtol=0, atol=1e-7)
    np.testing.assert_allclose(sampler.flow_sigmas(3, 1.0, 0.6), [0.75, 0.5, 0.25, 0.0], rtol=0, atol=1e-7)
    np.testing.assert_allclose(sampler.flow_sigmas(1, 1.0, 0.2), [0.25, 0.0], rtol=0, atol=1e-7)
    np.testing.assert_allclose(sampler.schedule_sigmas("simple", 4, 1.0, 0.8), [1.0, 0.75, 0.5, 0.25, 0.0],
                               rtol=0, atol=1e-7)
    # the full-schedule test is float32 too: 0.99995 rounds above 0.9999f
    assert sampler.flow_sigmas(4, 1.0, 0.99995) == sampler.flow_sigmas(4, 1.0)


@pytest.mark.gpu
def test_euler_stopping_above_zero_hands_back_leftover_noise(gpu):
    """A schedule that stops at sigma_last in (0, 1) returns x / (1 - sigma_last) (engine/src/pipeline.cu:583-588).
    On a straight trajectory x(s) = s n + (1 - s) x0 Euler is exact, so the result is x0 + s / (1 - s) n."""
    g = torch.Generator().manual_seed(15)
    x0, n = torch.randn(16, 4, 6, generator=g), torch.randn(16, 4, 6, generator=g)
    vd = (n - x0).to(DEV)

    def model(outs, xx, t, cfg_now):
        outs[0].copy_(vd)

    sig = sampler.flow_sigmas(6, 3.0)[:4]
    s = sig[-1]
    assert 0 < s < 1
    x = torch.empty(16, 4, 6, device=DEV)
    sampler.sample_euler(model, x, n.to(DEV), sig, negative=False)
    np.testing.assert_allclose(x.cpu().numpy(), (x0 + s / (1 - s) * n).numpy(), rtol=0, atol=5e-5)


@pytest.mark.gpu
def test_masked_euler_is_bit_identical_with_a_full_mask(gpu):
    """With mask 1 everywhere the masked Euler path computes the reference's k_euler_step expression on the same
    denoised values as the unmasked path (engine/src/pipeline.cu:326-331), so the results are bit-identical."""
    g = torch.Generator().manual_seed(16)
    init, n = torch.randn(16, 4, 6, generator=g).to(DEV), torch.randn(16, 4, 6, generator=g).to(DEV)

    def model(outs, xx, t, cfg_now):
        outs[0].copy_(0.7 * xx - 0.3 * init)

    sig = sampler.flow_sigmas(5, 3.0, 0.8)
    ref, x1 = torch.empty_like(init), torch.empty_like(init)
    sampler.sample_euler(model, ref, n, sig, negative=False, init=init)
    sampler.sample_euler(model, x1, n, sig, negative=False, init=init, mask=torch.ones(4, 6, device=DEV))
    assert torch.equal(x1, ref)


@pytest.mark.gpu
def test_ersde_trajectory_against_float64(gpu):
    """The er_sde loop (engine/src/pipeline.cu:481-482, 538-547) on a constant-velocity model against a float64
    statement of it: x starts at sigma_0 = 1 exactly (x = noise), then sigma_0 is clamped to float32(1 - 1e-4f)
    for the coefficients; stages 1-3 use the previous denoised values and first differences; the last step
    goes to the denoised estimate; noise torch_randn(seed + 1 + i)."""
    g = torch.Generator().manual_seed(17)
    x0, n = torch.randn(16, 4, 6, generator=g), torch.randn(16, 4, 6, generator=g)
    vd = (n - x0).to(DEV)

    def model(outs, xx, t, cfg_now):
        outs[0].copy_(vd)

    sig = sampler.flow_sigmas(6, 3.0)
    assert sig[0] == 1.0
    x = torch.empty(16, 4, 6, device=DEV)
    sampler.sample_euler(model, x, n.to(DEV), sig, negative=False, sampler="er_sde", seed=9)

    sc = list(sig)
    sc[0] = float(np.float32(1) - np.float32(1e-4))
    xr, v = n.double().clone(), (n - x0).double()
    old = oldd = None
    for i in range(6):
        den = xr - v * sc[i]
        if sc[i + 1] == 0.0:
            xr = den
            break
        a, b, c2, inv2, c3, inv3, cn, stage = sampler.ersde_coef(sc, i)
        nz = kiln_amd.torch_randn(9 + 1 + i, xr.numel()).view_as(xr).double()
        xn = a * xr + b * den
        if stage >= 2:
            d1 = (den - old) * inv2
            xn = xn + c2 * d1
            if stage >= 3:
                xn = xn + c3 * (d1 - oldd) * inv3
            oldd = d1
        xr = xn + cn * nz
        old = den
    np.testing.assert_allclose(x.cpu().double().numpy(), xr.numpy(), rtol=0, atol=1e-4)
