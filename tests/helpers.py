"""Shared helpers of the parity tests: seeded inputs and the error metrics of the tolerance bar."""
import numpy as np

# BASELINE tolerance against the fp32 (here: double-accumulation) reference
MAX_ABS = 2e-3
MEAN_ABS = 2e-4


def randn(seed, *shape, scale=1.0):
    """torch.manual_seed(seed); torch.randn(shape) on the CPU (== the reference's torch_randn)."""
    import torch
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g) * scale


def f16_round(t):
    """fp32 tensor holding exactly the fp16-representable values of t."""
    import torch
    return t.to(torch.float16).to(torch.float32)


def errors(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    d = np.abs(got - ref)
    rel_l2 = np.sqrt((d ** 2).sum() / max((ref ** 2).sum(), 1e-300))
    return float(d.max()), float(d.mean()), float(rel_l2)


def assert_close(got, ref, what, max_abs=MAX_ABS, mean_abs=MEAN_ABS):
    mx, mn, rl = errors(got, ref)
    print(f"[parity] {what}: max-abs {mx:.3e}  mean-abs {mn:.3e}  rel_l2 {rl:.3e}", flush=True)
    assert np.isfinite(np.asarray(got)).all(), f"{what}: non-finite output"
    assert mx <= max_abs, f"{what}: max-abs {mx:.3e} > {max_abs}"
    assert mn <= mean_abs, f"{what}: mean-abs {mn:.3e} > {mean_abs}"
    return mx, mn, rl
