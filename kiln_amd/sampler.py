"""Flow-matching Euler sampling with CFG for the DiT (the reference's sample(), engine/src/pipeline.cu:415-552,
for sampler "euler", scheduler "simple", no inpainting mask, no step cache).

Per step i with sigma s = sigmas[i]: the model sees timestep s * timestep_mult; while i < ceil(cfg_until *
steps) the prompt and the negative context run as one CFG batch and v = vn + cfg (v - vn) (kiln_cfg_combine);
then x advances by one Euler step to sigmas[i + 1] (kiln_flow_euler_step). x starts at sigmas[0] * noise
(+ (1 - sigmas[0]) * init for img2img). Every array operation runs on the GPU through the library.
"""
import math

import numpy as np

from . import (cfg_combine, flow_denoised, flow_denoised_masked, flow_ersde_step, flow_euler_den, flow_euler_step,
               flow_inpaint_in, flow_start, flow_update, torch_randn)


def flow_sigmas(steps, shift=1.0, denoise=1.0):
    """The "simple" schedule over ModelSamplingDiscreteFlow (engine/src/pipeline.cu:66-78): 1000 shifted sigmas
    t' = shift t / (1 + (shift - 1) t), t = (i + 1) / 1000, sampled every 1000 / total entries from the top,
    then 0; the last steps + 1 values (total = steps / denoise for partial denoising)."""
    total = steps if not _denoise_partial(denoise) else _denoise_total(steps, denoise)
    t = (np.arange(1000, dtype=np.float32) + np.float32(1)) / np.float32(1000)
    shift = np.float32(shift)
    table = t if shift == 1 else (shift * t / (np.float32(1) + (shift - np.float32(1)) * t)).astype(np.float32)
    ss = 1000.0 / total
    s = [float(table[999 - int(x * ss)]) for x in range(total)] + [0.0]
    return s[len(s) - (steps + 1):]


def _denoise_partial(denoise):
    """denoise > 0.9999f in the reference's float32 (pipeline.cu:67, 266): False means the full schedule."""
    return not (np.float32(denoise) > np.float32(0.9999))


def _denoise_total(steps, denoise):
    """(int)((double)steps / (double)denoise) with the reference's float32 denoise (pipeline.cu:67, 268)."""
    return int(float(steps) / float(np.float32(denoise)))


SAMPLERS = ("euler", "euler_ancestral", "dpmpp_2m", "res_multistep", "er_sde")
SCHEDULERS = ("simple", "normal", "sgm_uniform", "karras", "exponential", "ddim_uniform", "beta", "linear_quadratic",
              "kl_optimal")


def _snr_shift(shift, t):
    return t if shift == 1.0 else shift * t / (1.0 + (shift - 1.0) * t)


def _flow_table(shift):
    t = (np.arange(1000, dtype=np.float32) + np.float32(1)) / np.float32(1000)
    sh = np.float32(shift)
    return t if shift == 1.0 else (sh * t / (np.float32(1) + (sh - np.float32(1)) * t)).astype(np.float32)


def _full_schedule(name, steps, shift):
    """The ComfyUI schedulers over ModelSamplingDiscreteFlow(shift) (engine/src/pipeline.cu:188-262, flow space:
    timestep(sigma) = sigma, sigma(t) = shift t / (1 + (shift - 1) t), table[i] = sigma((i + 1) / 1000))."""
    tab = _flow_table(shift)
    f32 = lambda v: float(np.float32(v))  # noqa: E731  (the reference stores float32)
    smin, smax = float(tab[0]), float(tab[999])
    if name == "simple":
        ss = 1000.0 / steps
        return [float(tab[999 - int(x * ss)]) for x in range(steps)] + [0.0]
    if name in ("normal", "sgm_uniform"):
        start, end, n, zero = smax, smin, steps, True
        if name == "sgm_uniform":
            ts = [start + (end - start) * i / n for i in range(n + 1)][:-1]
        else:
            if abs(_snr_shift(shift, end)) < 1e-5:
                n, zero = n + 1, False
            ts = [start if n == 1 else start + (end - start) * i / (n - 1) for i in range(n)]
        return [f32(_snr_shift(shift, t)) for t in ts] + ([0.0] if zero else [])
    if name == "karras":
        a, b = smax ** (1 / 7.0), smin ** (1 / 7.0)
        return [f32((a + (0.0 if steps == 1 else i / (steps - 1)) * (b - a)) ** 7.0) for i in range(steps)] + [0.0]
    if name == "exponential":
        la, lb = math.log(smax), math.log(smin)
        return [f32(math.exp(la if steps == 1 else la + (lb - la) * i / (steps - 1))) for i in range(steps)] + [0.0]
    if name == "ddim_uniform":
        x, n, sig = 1, steps, []
        if abs(float(tab[x])) < 1e-5:
            n += 1
        else:
            sig.append(0.0)
        ss = max(1000 // n, 1)
        while x < 1000:
            sig.append(float(tab[x]))
            x += ss
        return sig[::-1]
    if name == "beta":
        from scipy.special import betaincinv  # the Beta(0.6, 0.6) quantile (the reference's beta_ppf)
        out, last = [], -1
        for i in range(steps):
            t = int(np.rint(betaincinv(0.6, 0.6, 1.0 - i / steps) * 999.0))
            if t != last:
                out.append(float(tab[t]))
            last = t
        return out + [0.0]
    if name == "linear_quadratic":
        if steps == 1:
            return [1.0, 0.0]
        thr, lin = 0.025, steps // 2
        quad = steps - lin
        sch = [i * thr / lin for i in range(lin)]
        diff = lin - thr * steps
        qc = diff / (lin * quad * quad)
        lc = thr / lin - 2 * diff / (quad * quad)
        cst = qc * lin * lin
        sch += [qc * i * i + lc * i + cst for i in range(lin, steps)] + [1.0]
        return [f32((1.0 - v) * smax) for v in sch]
    if name == "kl_optimal":
        return [f32(math.tan((0.0 if steps == 1 else i / (steps - 1)) * math.atan(smin) +
                             (1 - (0.0 if steps == 1 else i / (steps - 1))) * math.atan(smax)))
                for i in range(steps)] + [0.0]
    raise ValueError(f"unknown scheduler {name}")


def schedule_sigmas(name, steps, shift=1.0, denoise=1.0):
    """schedule_sigmas (engine/src/pipeline.cu:265-277): the schedule of steps / denoise steps, last steps + 1."""
    if not _denoise_partial(denoise):
        return _full_schedule(name, steps, shift)
    if np.float32(denoise) <= 0:
        return []
    s = _full_schedule(name, _denoise_total(steps, denoise), shift)
    return s if len(s) < steps + 1 else s[len(s) - (steps + 1):]


def step_coef(sampler, sig, i, have_old):
    """(a, b, c) of the step x <- a x + b den + c old from sigma_i to sigma_{i+1} (engine/src/pipeline.cu:396-411):
    first order (Euler) without history or at sigma 0; dpmpp_2m and res_multistep (eta 0) in log-sigma time."""
    s, sn = float(sig[i]), float(sig[i + 1])
    if sampler == "euler" or not have_old or sn == 0.0:
        return sn / s, 1.0 - sn / s, 0.0
    t, tn, tp = -math.log(s), -math.log(sn), -math.log(float(sig[i - 1]))
    h = tn - t
    if sampler == "dpmpp_2m":
        r = (t - tp) / h
        b = -math.expm1(-h)
        return sn / s, b * (1.0 + 1.0 / (2.0 * r)), -b / (2.0 * r)
    c2 = (tp - t) / h
    phi1 = math.expm1(-h) / (-h)
    phi2 = (phi1 - 1.0) / (-h)
    return math.exp(-h), h * (phi1 - phi2 / c2), h * (phi2 / c2)


def ersde_coef(sig, i):
    """Coefficients of the er_sde step from sigma_i to sigma_{i+1} (engine/src/pipeline.cu:361-391): lambda =
    sigma / (1 - sigma), noise scaler f(l) = l (exp(l^0.3) + 10), the integrals of 1/f and (l - l_i)/f over
    [l_{i+1}, l_i] by a 200-point left sum; stage min(3, i + 1). Returns (a, b, c2, inv2, c3, inv3, cn, stage)."""
    def lam(k):
        return sig[k] / (1.0 - sig[k])

    def f(l):
        return l * (math.exp(l ** 0.3) + 10.0)

    ls, lt = lam(i), lam(i + 1)
    as_, at = sig[i] / ls, sig[i + 1] / lt
    r, ra = f(lt) / f(ls), at / as_
    stage = min(3, i + 1)
    a, b, c2, inv2, c3, inv3 = ra * r, at * (1.0 - r), 0.0, 0.0, 0.0, 0.0
    if stage >= 2:
        dt = lt - ls
        step = -dt / 200.0
        S = Su = 0.0
        for k in range(200):
            lp = lt + k * step
            fp = f(lp)
            S += 1.0 / fp
            Su += (lp - ls) / fp
        S *= step
        Su *= step
        c2 = at * (dt + S * f(lt))
        inv2 = 1.0 / (ls - lam(i - 1))
        if stage >= 3:
            c3 = at * (dt * dt / 2.0 + Su * f(lt))
            inv3 = 2.0 / (ls - lam(i - 2))
    cn = at * math.sqrt(max(0.0, lt * lt - ls * ls * r * r))
    return a, b, c2, inv2, c3, inv3, cn, stage


def initial_noise(seed, shape, device):
    """The sampler's noise (engine/src/pipeline.cu:428-429): torch_randn(seed, n) on the host, then to the device."""
    from . import torch_randn
    n = 1
    for d in shape:
        n *= d
    return torch_randn(seed, n).view(*shape).to(device)


def sample_euler(model, x, noise, sigmas, cfg=1.0, cfg_until=1.0, timestep_mult=1.0, init=None, negative=True,
                 cache=None, cache_start=0.15, cache_end=0.9, cache_max_hits=2, sampler="euler", seed=0, mask=None):
    """model(outs, x, t, cfg_now) writes the velocity of the prompt into outs[0] and, when cfg_now, of the
    negative context into outs[1]; x [16, Hl, Wl] fp32 (overwritten with the result), noise like x;
    negative: whether a negative context exists (CFG runs for the first ceil(cfg_until * steps) steps).
    sampler: "euler" (k_euler_step's arithmetic), "euler_ancestral" (the RF ancestral step with eta 1, fresh
    noise torch_randn(seed + 1 + i) per step, pipeline.cu:514-529), "dpmpp_2m" or "res_multistep" (step_coef),
    "er_sde" (ersde_coef, up to third order, same per-step noise, pipeline.cu:538-547).
    mask: inpainting mask [Hl, Wl] (1 = regenerate) with init: the model sees the init re-noised to each sigma
    outside the mask and the denoised estimate is pinned to the init there (pipeline.cu:309-324, 485, 512).
    cache: a kiln_amd.dit.StepCache the model's forward uses, or None; the sampler allows a skip only after the
    first max(2, ceil(cache_start * steps)) steps, before the last max(1, ceil((1 - cache_end) * steps)), and
    for at most cache_max_hits steps in a row (engine/src/pipeline.cu:463-480, 488, 506-509). Returns x; the
    number of skipped steps is in cache.skips."""
    import torch
    steps = len(sigmas) - 1
    if steps < 1:
        if init is not None:
            x.copy_(init)
        return x
    if sampler not in SAMPLERS:
        raise ValueError(f"unknown sampler {sampler}")
    v, vn = torch.empty_like(x), torch.empty_like(x)
    den, old = torch.empty_like(x), torch.empty_like(x)
    have_old = False
    if mask is not None and init is None:
        raise ValueError("an inpainting mask needs init")
    xin = torch.empty_like(x) if mask is not None else x
    sigmas = list(sigmas)
    if sampler == "er_sde":
        oldd = torch.empty_like(x)
    cfg_steps = math.ceil(cfg_until * steps - 1e-4) if negative else 0
    warm = max(2, math.ceil(cache_start * steps))
    tail = max(1, math.ceil((1.0 - cache_end) * steps))
    max_hits = steps if cache_max_hits < 0 else cache_max_hits
    run = 0
    if cache is not None:
        cache.skips = 0
    flow_start(x, noise, sigmas[0], init)
    if sampler == "er_sde" and np.float32(sigmas[0]) >= 1:
        # lambda = sigma / (1 - sigma) needs sigma < 1; the start above used the unclamped sigma
        # (pipeline.cu:481-482), the clamp is float32 1 - 1e-4f
        sigmas[0] = float(np.float32(1) - np.float32(1e-4))
    for i in range(steps):
        s = sigmas[i]
        cfg_now = i < cfg_steps
        if cache is not None:
            cache.allow = warm <= i < steps - tail and run < max_hits
        if mask is not None:
            flow_inpaint_in(xin, x, noise, init, mask, s)
        model([v, vn], xin, s * timestep_mult, cfg_now)
        if cache is not None:
            if cache.skipped:
                cache.skips += 1
                run += 1
            else:
                run = 0
        if cfg_now:
            cfg_combine(v, vn, cfg)
        sn = sigmas[i + 1]
        if mask is not None:  # every sampler goes through the pinned denoised estimate
            flow_denoised_masked(den, xin, v, init, mask, s)
        if sampler == "euler" and mask is None:
            flow_euler_step(x, v, s, sn)
        elif sampler == "euler":
            flow_euler_den(x, den, s, sn)
        elif sampler == "er_sde":
            if mask is None:
                flow_denoised(den, x, v, s)
            if sn == 0.0:
                flow_update(x, den, 0.0, 1.0)
            else:
                nz = torch_randn(seed + 1 + i, x.numel()).view_as(x).to(x.device)
                flow_ersde_step(x, den, old, oldd, nz, ersde_coef(sigmas, i))
        elif sampler == "euler_ancestral":
            if mask is None:
                flow_denoised(den, x, v, s)
            if sn == 0.0:
                flow_update(x, den, 0.0, 1.0)
            else:
                sd = sn * (1.0 + (sn / s - 1.0))
                aip1, ad = 1.0 - sn, 1.0 - sd
                renoise = math.sqrt(max(0.0, sn * sn - sd * sd * aip1 * aip1 / (ad * ad)))
                r, a = sd / s, aip1 / ad
                flow_update(x, den, a * r, a * (1.0 - r))
                nz = torch_randn(seed + 1 + i, x.numel()).view_as(x).to(x.device)
                flow_update(x, nz, 1.0, renoise)
        else:
            if mask is None:
                flow_denoised(den, x, v, s)
            a, b, c = step_coef(sampler, sigmas, i, have_old)
            flow_update(x, den, a, b, old if have_old else None, c)
        if sampler != "euler" or mask is not None:
            den, old = old, den
            have_old = True
    last = float(np.float32(sigmas[-1]))
    if 0.0 < last < 1.0:
        # stopped above sigma 0 (leftover noise for a second pass): x / (1 - sigma) (pipeline.cu:583-588)
        flow_update(x, x, float(np.float32(1) / (np.float32(1) - np.float32(last))), 0.0)
    return x
