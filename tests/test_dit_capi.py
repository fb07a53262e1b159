"""libkiln_dit.so on the CPU (no kernel launched): it loads, exports every symbol include/kiln_dit.h declares (all
bound in the Python binding), its host arithmetic (schedules, the beta scheduler's quantile, sampler
coefficients) against closed forms and an independent library, and its argument checks."""
import ctypes
import math
import os

import numpy as np
import pytest

import kiln_amd
from kiln_amd import dit, sampler

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "kiln_dit.h")


def test_exports_every_header_symbol():
    L = dit.dlib()
    syms = kiln_amd.header_symbols(HEADER)
    assert len(syms) >= 20
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, f"declared in include/kiln_dit.h but not exported: {missing}"
    assert sorted(dit._SIGS) == syms


def test_beta_quantile_closed_forms_and_scipy():
    """The beta scheduler's Beta(0.6, 0.6) quantile (pipeline.cu:124-137): Beta(1, 1) is uniform (ppf = p),
    Beta(1/2, 1/2) is the arcsine law (ppf = sin^2(pi p / 2)), Beta(2, 1) has ppf = sqrt(p); Beta(0.6, 0.6)
    against scipy's betaincinv (an independent implementation)."""
    from scipy.special import betaincinv
    for p in np.linspace(0.0005, 0.9995, 101):
        assert abs(sampler.beta_quantile(p, 1, 1) - p) < 1e-13
        assert abs(sampler.beta_quantile(p, 0.5, 0.5) - math.sin(math.pi * p / 2) ** 2) < 1e-13
        assert abs(sampler.beta_quantile(p, 2, 1) - math.sqrt(p)) < 1e-13
        assert abs(sampler.beta_quantile(p, 0.6, 0.6) - betaincinv(0.6, 0.6, p)) < 1e-12
    assert sampler.beta_quantile(0.0, 0.6, 0.6) == 0.0 and sampler.beta_quantile(1.0, 0.6, 0.6) == 1.0


def test_beta_schedule_indices():
    """The beta schedule takes table entries at round(ppf(1 - i/steps) * 999), merging repeats, then 0."""
    from scipy.special import betaincinv
    for shift in (1.0, 3.0):
        t = np.arange(1, 1001, dtype=np.float32) / np.float32(1000)
        tab = t if shift == 1.0 else (np.float32(shift) * t / (1 + np.float32(shift - 1) * t)).astype(np.float32)
        for steps in (4, 9, 20, 40):
            idx = [int(np.rint(betaincinv(0.6, 0.6, 1 - i / steps) * 999)) for i in range(steps)]
            keep = [k for j, k in enumerate(idx) if j == 0 or k != idx[j - 1]]
            assert sampler.schedule_sigmas("beta", steps, shift) == [float(tab[k]) for k in keep] + [0.0]


def test_schedules_reject_unknown_and_bad():
    with pytest.raises(kiln_amd.KilnError):
        sampler.schedule_sigmas("no_such_scheduler", 8)
    with pytest.raises(kiln_amd.KilnError):
        sampler.schedule_sigmas("karras", 0)
    assert sampler.schedule_sigmas("karras", 8, 3.0, 0.0) == []


def test_ersde_coefficients_match_a_double_statement():
    """er_sde (pipeline.cu:361-391): lambda = s / (1 - s), f(l) = l (exp(l^0.3) + 10); a = alpha'/alpha r,
    b = alpha'(1 - r), r = f(l')/f(l), noise scale alpha' sqrt(l'^2 - l^2 r^2); the stage-2/3 integrals by a
    fine trapezoid rule (the library's 200-point left sum must agree to its own truncation error)."""
    sig = sampler.flow_sigmas(10, 3.0)
    sig[0] = float(np.float32(1) - np.float32(1e-4))
    lam = [s / (1 - s) if s < 1 else float("inf") for s in sig]
    f = lambda l: l * (math.exp(l ** 0.3) + 10.0)  # noqa: E731
    for i in range(9):
        a, b, c2, inv2, c3, inv3, cn, stage = sampler.ersde_coef(sig, i)
        ls, lt = lam[i], lam[i + 1]
        r = f(lt) / f(ls)
        at, as_ = sig[i + 1] / lt, sig[i] / ls
        assert stage == min(3, i + 1)
        assert abs(a - at / as_ * r) <= 1e-6 * abs(at / as_ * r) + 1e-9
        assert abs(b - at * (1 - r)) <= 1e-6 * abs(at * (1 - r)) + 1e-9
        assert abs(cn - at * math.sqrt(max(0.0, lt * lt - ls * ls * r * r))) <= 1e-5 * abs(cn) + 1e-9
        if stage >= 2:
            xs = np.linspace(lt, ls, 20001)
            S = np.trapezoid([1 / f(x) for x in xs], xs)  # integral of 1/f over [l', l]
            ref_c2 = at * ((lt - ls) + S * f(lt))
            assert abs(c2 - ref_c2) <= 0.02 * abs(ref_c2) + 1e-7, (i, c2, ref_c2)
            assert abs(inv2 - 1 / (ls - lam[i - 1])) <= 1e-6 * abs(inv2)


def test_argument_checks_return_before_any_gpu_call():
    L = dit.dlib()
    out = ctypes.c_void_p()
    assert L.kiln_dit_create(None, None, ctypes.byref(out)) == kiln_amd.KILN_EINVAL
    assert b"null" in L.kiln_dit_last_error()
    bad = dit.Dims(2, 3, 1024, 0, 1e-6)  # odd head count
    assert L.kiln_dit_create(ctypes.byref(bad), None, ctypes.byref(out)) == kiln_amd.KILN_EINVAL
    assert b"unsupported" in L.kiln_dit_last_error()
    abc = (ctypes.c_float * 3)()
    sig = (ctypes.c_float * 2)(1.0, 0.0)
    assert L.kiln_step_coef(b"euler", sig, 2, 1, 0, abc) == kiln_amd.KILN_EINVAL  # i + 1 beyond the schedule
    assert L.kiln_step_coef(b"euler", sig, 2, 0, 0, abc) == 0 and abs(abc[0]) < 1e-12 and abs(abc[1] - 1) < 1e-7


def test_device_failures_keep_their_status():
    """A HIP failure inside the driver comes back as KILN_EHIP, not as a bad argument: on a machine without a GPU
    caching a context fails in its first hipMalloc (the C ABI maps the driver's typed errors to their status)."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("needs a machine without a GPU")
    L = dit.dlib()
    out = ctypes.c_void_p()
    assert L.kiln_dit_create(ctypes.byref(dit.Dims(2, 4, 1024, 512, 1e-6)), None, ctypes.byref(out)) == 0
    try:
        buf = (ctypes.c_float * 4096)()
        ctx = ctypes.c_void_p()
        assert L.kiln_dit_cache_context(out, buf, 1, 1, 0, ctypes.byref(ctx)) == kiln_amd.KILN_EHIP
        assert b"hipMalloc" in L.kiln_dit_last_error()
    finally:
        L.kiln_dit_destroy(out)


def test_engine_reports_fatal_without_a_device():
    """kiln_engine's start-up failure path (main.cpp:647-660: a fatal event, exit code 1), on a machine without
    a GPU; the protocol itself is tested on the GPU (tests/test_engine_protocol_gpu.py)."""
    import subprocess
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    exe = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "kiln_amd", "kiln_engine")
    r = subprocess.run([exe], input='{"cmd":"info","id":"x"}\n', capture_output=True, text=True, timeout=60)
    import json
    ev = [json.loads(ln) for ln in r.stdout.splitlines() if ln.strip()]
    assert r.returncode == 1 and ev and ev[-1]["ev"] == "fatal" and ev[-1]["msg"]
