"""Python binding of the flow-matching sampler (libkiln_dit.so: kiln_amd/host/sampler.cpp): the reference's
sample() (engine/src/pipeline.cu:415-598) with its samplers, schedulers (pipeline.cu:66-78, 188-277) and step
coefficients (pipeline.cu:361-411). The schedules, coefficients and the loop run in C++; every array operation
runs on the GPU. sample_euler drives a Python velocity model through a C callback; kiln_amd.dit.Dit.sample
drives the DiT without leaving C++.
"""
import ctypes

import numpy as np

from .dit import STEP_FN, VELOCITY_FN, SampleParams, _check, _f32, dlib

SAMPLERS = ("euler", "euler_ancestral", "dpmpp_2m", "res_multistep", "er_sde")
SCHEDULERS = ("simple", "normal", "sgm_uniform", "karras", "exponential", "ddim_uniform", "beta", "linear_quadratic",
              "kl_optimal")


def schedule_sigmas(name, steps, shift=1.0, denoise=1.0):
    """schedule_sigmas (engine/src/pipeline.cu:265-277): the last steps + 1 sigmas of the schedule of
    (int)(steps / denoise) steps (denoise as float32), ending in 0; [] for denoise <= 0."""
    cap = 4 * max(int(steps), 1) + 1100
    buf = (ctypes.c_float * cap)()
    n = dlib().kiln_schedule_sigmas(name.encode(), int(steps), float(shift), float(denoise), buf, cap)
    if n < 0:
        _check(-n)
    return [float(v) for v in np.frombuffer(buf, np.float32)[:n]]


def flow_sigmas(steps, shift=1.0, denoise=1.0):
    """The "simple" schedule over ModelSamplingDiscreteFlow (engine/src/pipeline.cu:66-78)."""
    return schedule_sigmas("simple", steps, shift, denoise)


def _sig(sig):
    a = np.ascontiguousarray(np.asarray(sig, dtype=np.float32))
    return a, a.ctypes.data_as(ctypes.c_void_p)


def step_coef(sampler, sig, i, have_old):
    """(a, b, c) of the step x <- a x + b den + c old from sigma_i to sigma_{i+1} (pipeline.cu:396-411)."""
    a, p = _sig(sig)
    out = (ctypes.c_float * 3)()
    _check(dlib().kiln_step_coef(sampler.encode(), p, len(a), int(i), int(bool(have_old)), out))
    return tuple(float(v) for v in out)


def ersde_coef(sig, i):
    """The er_sde step's coefficients (a, b, c2, inv2, c3, inv3, cn, stage) (pipeline.cu:361-391)."""
    a, p = _sig(sig)
    out = (ctypes.c_float * 7)()
    stage = ctypes.c_int()
    _check(dlib().kiln_ersde_coef(p, len(a), int(i), out, ctypes.byref(stage)))
    return tuple(float(v) for v in out) + (stage.value,)


def beta_quantile(p, a, b):
    """The Beta(a, b) quantile of the beta scheduler."""
    return dlib().kiln_beta_quantile(float(p), float(a), float(b))


def initial_noise(seed, shape, device):
    """The sampler's noise (engine/src/pipeline.cu:428-429): torch_randn(seed, n) on the host, then to the device."""
    from . import torch_randn
    n = 1
    for d in shape:
        n *= d
    return torch_randn(seed, n).view(*shape).to(device)


def make_params(x, steps=8, cfg=1.0, shift=3.0, denoise=1.0, seed=0, cfg_until=1.0, sampler="euler",
                scheduler="simple", sigmas=None, add_noise=True, noise=None, timestep_mult=1.0, cache_threshold=0.0,
                cache_start=0.15, cache_end=0.9, cache_max_hits=2):
    """kiln_sample_params for a latent like x; returns (params, objects the params point into)."""
    sp = SampleParams()
    dlib().kiln_sample_params_default(ctypes.byref(sp))
    keep = []
    sp.steps, sp.cfg, sp.shift, sp.denoise, sp.seed, sp.cfg_until = steps, cfg, shift, denoise, seed, cfg_until
    for name, v in (("sampler", sampler), ("scheduler", scheduler)):
        b = v.encode()
        keep.append(b)
        setattr(sp, name, b)
    if sigmas is not None:
        a, p = _sig(sigmas)
        keep.append(a)
        sp.sigmas, sp.nsigmas = p, len(a)
    sp.add_noise = int(bool(add_noise))
    if noise is not None:
        h = np.ascontiguousarray(noise.detach().float().cpu().numpy().reshape(-1))
        if h.size != x.numel():
            raise ValueError(f"noise has {h.size} elements, the latent {x.numel()}")
        keep.append(h)
        sp.noise = h.ctypes.data_as(ctypes.c_void_p)
    sp.timestep_mult = timestep_mult
    sp.cache_threshold, sp.cache_start, sp.cache_end, sp.cache_max_hits = (cache_threshold, cache_start, cache_end,
                                                                          cache_max_hits)
    return sp, keep


class _DeviceArray:
    """A float32 device buffer of the given shape as a __cuda_array_interface__ view (for torch.as_tensor)."""

    def __init__(self, ptr, shape):
        self.__cuda_array_interface__ = {"shape": tuple(shape), "typestr": "<f4", "data": (ptr, False),
                                         "version": 2, "strides": None}


def sample_euler(model, x, noise, sigmas, cfg=1.0, cfg_until=1.0, timestep_mult=1.0, init=None, negative=True,
                 cache=None, cache_start=0.15, cache_end=0.9, cache_max_hits=2, sampler="euler", seed=0, mask=None,
                 stream=None):
    """sample() (engine/src/pipeline.cu:415-598) with a Python velocity model, on the explicit schedule `sigmas`.
    model(outs, x, t, cfg_now) writes the prompt's velocity into outs[0] and, when cfg_now, the negative context's
    into outs[1] (torch views of the sampler's device buffers, shaped like x); x [16, Hl, Wl] fp32 (overwritten
    with the result); noise like x (the start noise); negative: a negative context exists (CFG for the first
    ceil(cfg_until * steps) steps); init: img2img start; mask [Hl, Wl] (1 = regenerate) with init: inpainting;
    sampler: euler, euler_ancestral, dpmpp_2m, res_multistep, er_sde (per-step noise torch_randn(seed + 1 + i));
    cache: an object with `threshold`, `allow`, `skipped`, `skips` (kiln_amd.dit.StepCache or a stand-in) whose
    `allow` the sampler sets per step under the reference's guards; its `skips` counts the skipped steps. Returns x.
    """
    import torch
    if sampler not in SAMPLERS:
        raise ValueError(f"unknown sampler {sampler}")
    if len(sigmas) < 2:  # nothing to do (denoise 0): the result is the input
        if init is not None:
            x.copy_(init)
        return x
    Hl, Wl = x.shape[-2], x.shape[-1]
    n = 16 * Hl * Wl
    if mask is not None and tuple(mask.shape[-2:]) != (Hl, Wl):
        raise ValueError(f"mask of shape {tuple(mask.shape)} does not match the latent's {Hl} x {Wl}")
    thr = float(cache.threshold) if cache is not None else 0.0
    sp, keep = make_params(x, sigmas=sigmas, cfg=cfg, cfg_until=cfg_until, timestep_mult=timestep_mult, noise=noise,
                           sampler=sampler, seed=seed, cache_threshold=thr, cache_start=cache_start,
                           cache_end=cache_end, cache_max_hits=cache_max_hits)
    shape = tuple(x.shape)
    err = []

    def velocity(user, outs, xp, t, cfg_now, allow, skipped):
        try:
            view = lambda p: torch.as_tensor(_DeviceArray(p, shape), device=x.device)  # noqa: E731
            o = [view(outs[0]), view(outs[1]) if cfg_now else None]
            if cache is not None:
                cache.allow = bool(allow)
            model(o, view(xp), t, bool(cfg_now))
            skipped[0] = int(bool(cache.skipped)) if cache is not None else 0
            return 0
        except Exception as e:  # re-raised below
            err.append(e)
            return 1

    cb = VELOCITY_FN(velocity)
    skips = ctypes.c_int(0)
    s = stream if stream is not None else torch.cuda.current_stream()
    rc = dlib().kiln_sample(cb, None, _f32(x, n, "x"), Hl, Wl, int(bool(negative)), ctypes.byref(sp),
                            _f32(init, n, "init") if init is not None else None,
                            _f32(mask, Hl * Wl, "mask") if mask is not None else None, STEP_FN(), None, None,
                            ctypes.byref(skips), ctypes.c_void_p(s.cuda_stream))
    if err:
        raise err[0]
    _check(rc)
    if cache is not None:
        cache.skips = skips.value
    del keep
    return x
