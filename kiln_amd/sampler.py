"""Flow-matching Euler sampling with CFG for the DiT (the reference's sample(), engine/src/pipeline.cu:415-552,
for sampler "euler", scheduler "simple", no inpainting mask, no step cache).

Per step i with sigma s = sigmas[i]: the model sees timestep s * timestep_mult; while i < ceil(cfg_until *
steps) the prompt and the negative context run as one CFG batch and v = vn + cfg (v - vn) (kiln_cfg_combine);
then x advances by one Euler step to sigmas[i + 1] (kiln_flow_euler_step). x starts at sigmas[0] * noise
(+ (1 - sigmas[0]) * init for img2img). Every array operation runs on the GPU through the library.
"""
import math

import numpy as np

from . import cfg_combine, flow_euler_step, flow_start


def flow_sigmas(steps, shift=1.0, denoise=1.0):
    """The "simple" schedule over ModelSamplingDiscreteFlow (engine/src/pipeline.cu:66-78): 1000 shifted sigmas
    t' = shift t / (1 + (shift - 1) t), t = (i + 1) / 1000, sampled every 1000 / total entries from the top,
    then 0; the last steps + 1 values (total = steps / denoise for partial denoising)."""
    total = steps if denoise > 0.9999 else int(steps / denoise)
    t = (np.arange(1000, dtype=np.float32) + np.float32(1)) / np.float32(1000)
    shift = np.float32(shift)
    table = t if shift == 1 else (shift * t / (np.float32(1) + (shift - np.float32(1)) * t)).astype(np.float32)
    ss = 1000.0 / total
    s = [float(table[999 - int(x * ss)]) for x in range(total)] + [0.0]
    return s[len(s) - (steps + 1):]


def initial_noise(seed, shape, device):
    """The sampler's noise (engine/src/pipeline.cu:428-429): torch_randn(seed, n) on the host, then to the device."""
    from . import torch_randn
    n = 1
    for d in shape:
        n *= d
    return torch_randn(seed, n).view(*shape).to(device)


def sample_euler(model, x, noise, sigmas, cfg=1.0, cfg_until=1.0, timestep_mult=1.0, init=None, negative=True,
                 cache=None, cache_start=0.15, cache_end=0.9, cache_max_hits=2):
    """model(outs, x, t, cfg_now) writes the velocity of the prompt into outs[0] and, when cfg_now, of the
    negative context into outs[1]; x [16, Hl, Wl] fp32 (overwritten with the result), noise like x;
    negative: whether a negative context exists (CFG runs for the first ceil(cfg_until * steps) steps).
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
    v, vn = torch.empty_like(x), torch.empty_like(x)
    cfg_steps = math.ceil(cfg_until * steps - 1e-4) if negative else 0
    warm = max(2, math.ceil(cache_start * steps))
    tail = max(1, math.ceil((1.0 - cache_end) * steps))
    max_hits = steps if cache_max_hits < 0 else cache_max_hits
    run = 0
    if cache is not None:
        cache.skips = 0
    flow_start(x, noise, sigmas[0], init)
    for i in range(steps):
        s = sigmas[i]
        cfg_now = i < cfg_steps
        if cache is not None:
            cache.allow = warm <= i < steps - tail and run < max_hits
        model([v, vn], x, s * timestep_mult, cfg_now)
        if cache is not None:
            if cache.skipped:
                cache.skips += 1
                run += 1
            else:
                run = 0
        if cfg_now:
            cfg_combine(v, vn, cfg)
        flow_euler_step(x, v, s, sigmas[i + 1])
    return x
