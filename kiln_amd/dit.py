"""Python binding of the DiT step driver (libkiln_dit.so, include/kiln_dit.h): the Cosmos-Predict2 DiT forward,
its per-generation context cache, the first-block step cache and NAG, implemented in C++
(kiln_amd/host/dit.cpp) over the HIP library. The reference's Dit (engine/src/models.h:20-90,
engine/src/dit.cu:217-546).

    d = Dit(blocks=28, heads=16)                       # D = 128 * heads
    d.set_step_weights(t_lin1=..., ...)                # bf16 device tensors, [out, in]
    d.set_block(i, sa_q=..., ..., mod=[6 tensors])     # copied; linear weights converted to fp16 at load
    pos = d.cache_context(ctx)                         # ctx [len, ctx_dim] fp32 (Dit::cache_context)
    d.forward([v0, v1], latent, t, [pos, neg], nag=Nag(neg_ctx))   # Dit::forward_batch

Every call runs on the GPU through the library; there is no CPU path.
"""
import ctypes

import torch

from . import KILN_OK, KilnError, lib

_vp, _i, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
_DLIB = None


class Dims(ctypes.Structure):
    _fields_ = [("blocks", _i), ("heads", _i), ("ctx_dim", _i), ("mlp", _i), ("eps", _f)]


_BLOCK_FIELDS = ["sa_q", "sa_k", "sa_v", "sa_o", "ca_q", "ca_o", "ca_k", "ca_v", "mlp1", "mlp2", "sa_qn", "sa_kn",
                 "ca_qn", "ca_kn", "mod_sa1", "mod_sa2", "mod_ca1", "mod_ca2", "mod_mlp1", "mod_mlp2"]
_STEP_FIELDS = ["t_lin1", "t_lin2", "t_norm", "final_mod1", "final_mod2", "x_embed", "final_lin"]


class BlockWeights(ctypes.Structure):
    _fields_ = [(n, _vp) for n in _BLOCK_FIELDS]


class StepWeightsC(ctypes.Structure):
    _fields_ = [(n, _vp) for n in _STEP_FIELDS]


class NagC(ctypes.Structure):
    _fields_ = [("neg", _vp), ("scale", _f), ("tau", _f), ("alpha", _f)]


class SampleParams(ctypes.Structure):
    _fields_ = [("steps", _i), ("cfg", _f), ("shift", _f), ("denoise", _f), ("seed", ctypes.c_uint64),
                ("cfg_until", _f), ("sampler", ctypes.c_char_p), ("scheduler", ctypes.c_char_p), ("sigmas", _vp),
                ("nsigmas", _i), ("add_noise", _i), ("noise", _vp), ("timestep_mult", _f),
                ("cache_threshold", _f), ("cache_start", _f), ("cache_end", _f), ("cache_max_hits", _i)]


VELOCITY_FN = ctypes.CFUNCTYPE(_i, _vp, ctypes.POINTER(_vp), _vp, _f, _i, _i, ctypes.POINTER(_i))
STEP_FN = ctypes.CFUNCTYPE(None, _vp, _i, _i, _f, _vp, _vp, ctypes.c_double)

_SIGS = {
    "kiln_dit_create": (_i, [ctypes.POINTER(Dims), _vp, ctypes.POINTER(_vp)]),
    "kiln_dit_destroy": (None, [_vp]),
    "kiln_dit_set_step_weights": (_i, [_vp, ctypes.POINTER(StepWeightsC)]),
    "kiln_dit_set_block": (_i, [_vp, _i, ctypes.POINTER(BlockWeights)]),
    "kiln_dit_cache_context": (_i, [_vp, _vp, _i, _i, _i, ctypes.POINTER(_vp)]),
    "kiln_dit_context_destroy": (None, [_vp]),
    "kiln_dit_context_kv": (_i, [_vp, _i, ctypes.POINTER(_vp), ctypes.POINTER(_i), ctypes.POINTER(_i)]),
    "kiln_dit_step_cache_create": (_i, [_f, ctypes.POINTER(_vp)]),
    "kiln_dit_step_cache_destroy": (None, [_vp]),
    "kiln_dit_step_cache_set_allow": (_i, [_vp, _i]),
    "kiln_dit_step_cache_state": (_i, [_vp, ctypes.POINTER(_i), ctypes.POINTER(_i), ctypes.POINTER(_f)]),
    "kiln_dit_forward": (_i, [_vp, _vp, _vp, _i, _i, _f, _vp, _i, ctypes.POINTER(NagC), _vp, _i]),
    "kiln_dit_step_tables": (_i, [_vp, _f, _vp]),
    "kiln_dit_run_block": (_i, [_vp, _i, _vp, _vp, _i, _i, _vp, _i, ctypes.POINTER(NagC), _i]),
    "kiln_dit_last_error": (ctypes.c_char_p, []),
    "kiln_schedule_sigmas": (_i, [ctypes.c_char_p, _i, _f, _f, _vp, _i]),
    "kiln_step_coef": (_i, [ctypes.c_char_p, _vp, _i, _i, _i, _vp]),
    "kiln_ersde_coef": (_i, [_vp, _i, _i, _vp, ctypes.POINTER(_i)]),
    "kiln_beta_quantile": (ctypes.c_double, [ctypes.c_double, ctypes.c_double, ctypes.c_double]),
    "kiln_sample_params_default": (None, [ctypes.POINTER(SampleParams)]),
    "kiln_sample": (_i, [VELOCITY_FN, _vp, _vp, _i, _i, _i, ctypes.POINTER(SampleParams), _vp, _vp, STEP_FN, _vp,
                         _vp, ctypes.POINTER(_i), _vp]),
    "kiln_dit_sample": (_i, [_vp, _vp, _i, _i, _vp, _vp, ctypes.POINTER(NagC), _f, _i, _i,
                             ctypes.POINTER(SampleParams), _vp, _vp, STEP_FN, _vp, _vp, ctypes.POINTER(_i)]),
}


def dlib():
    """Load libkiln_dit.so (next to libkiln_attn.so; built by kiln_amd/build.py)."""
    global _DLIB
    if _DLIB is None:
        import os
        from . import LIB_PATH
        lib()  # libkiln_attn.so first: the driver links it
        path = os.path.join(os.path.dirname(LIB_PATH), "libkiln_dit.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: build it with `python -m kiln_amd.build`")
        L = ctypes.CDLL(path)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _DLIB = L
    return _DLIB


def _check(rc):
    if rc != KILN_OK:
        raise KilnError(rc, dlib().kiln_dit_last_error().decode())


def _p(t):
    return None if t is None else _vp(t.data_ptr())


def _bf16(t, n=None, name=""):
    if t is None:
        raise ValueError(f"missing weight {name}")
    if t.dtype != torch.bfloat16 or not t.is_contiguous() or not t.is_cuda:
        raise ValueError(f"weight {name}: expected a contiguous bf16 device tensor")
    if n is not None and t.numel() != n:
        raise ValueError(f"weight {name}: {t.numel()} elements, expected {n}")
    return _p(t)


def _f32(t, n=None, name=""):
    if t.dtype != torch.float32 or not t.is_contiguous() or not t.is_cuda:
        raise ValueError(f"{name}: expected a contiguous float32 device tensor")
    if n is not None and t.numel() != n:
        raise ValueError(f"{name}: {t.numel()} elements, expected {n}")
    return _p(t)


class _DevPtr:
    """A device address owned by another object (kept alive with it), with torch's data_ptr() spelling."""

    def __init__(self, addr, owner):
        self._addr, self._owner = addr, owner

    def data_ptr(self):
        return self._addr


class Context:
    """A text context cached for one generation (Dit::cache_context): real rows and the padded length."""

    def __init__(self, handle, real, length):
        self._h, self.real, self.len = handle, real, length

    @property
    def handle(self):
        return self._h

    def kv(self, block):
        """Block `block`'s prepared K/V (kiln_dit_context_kv): an object with data_ptr(), as the cross-attention
        entry points of kiln_amd take prepared buffers; valid while this context lives."""
        p, real, length = ctypes.c_void_p(), ctypes.c_int(), ctypes.c_int()
        _check(dlib().kiln_dit_context_kv(self._h, int(block), ctypes.byref(p), ctypes.byref(real),
                                          ctypes.byref(length)))
        return _DevPtr(p.value, self)

    def __del__(self):
        if getattr(self, "_h", None):
            dlib().kiln_dit_context_destroy(self._h)
            self._h = None


class Nag:
    """NAG on batch item 0 (Dit::Nag, engine/src/models.h:80)."""

    def __init__(self, neg, scale=5.0, tau=2.5, alpha=0.25):
        self.neg, self.scale, self.tau, self.alpha = neg, scale, tau, alpha

    def c(self):
        return NagC(self.neg.handle.value, self.scale, self.tau, self.alpha)


def _nag(nag):
    return ctypes.byref(nag.c()) if nag is not None else None


class StepCache:
    """The first-block step cache (Dit::StepCache, engine/src/models.h:66-76). `allow` is set per step by a
    sampler; after a forward, `skipped`, `valid` and `last_change` report what it did."""

    def __init__(self, threshold):
        h = _vp()
        _check(dlib().kiln_dit_step_cache_create(threshold, ctypes.byref(h)))
        self._h, self.threshold, self._allow, self.skips = h, threshold, False, 0

    @property
    def handle(self):
        return self._h

    @property
    def allow(self):
        return self._allow

    @allow.setter
    def allow(self, v):
        self._allow = bool(v)
        _check(dlib().kiln_dit_step_cache_set_allow(self._h, int(self._allow)))

    def _state(self):
        sk, va, lc = _i(), _i(), _f()
        _check(dlib().kiln_dit_step_cache_state(self._h, ctypes.byref(sk), ctypes.byref(va), ctypes.byref(lc)))
        return bool(sk.value), bool(va.value), lc.value

    @property
    def skipped(self):
        return self._state()[0]

    @property
    def valid(self):
        return self._state()[1]

    @property
    def last_change(self):
        return self._state()[2]

    def __del__(self):
        if getattr(self, "_h", None):
            dlib().kiln_dit_step_cache_destroy(self._h)
            self._h = None


class Dit:
    """The DiT on the current device (Dit, engine/src/models.h:20-90), GPU work on `stream` (torch's current
    stream by default)."""

    def __init__(self, blocks, heads, ctx_dim=1024, mlp=0, eps=1e-6, stream=None):
        self.blocks, self.heads, self.ctx_dim = blocks, heads, ctx_dim
        self.D = 128 * heads
        self.F = mlp if mlp else 4 * self.D
        self.eps = eps
        self._stream = stream if stream is not None else torch.cuda.current_stream()
        h = _vp()
        _check(dlib().kiln_dit_create(ctypes.byref(Dims(blocks, heads, ctx_dim, mlp, eps)),
                                      _vp(self._stream.cuda_stream), ctypes.byref(h)))
        self._h = h

    def __del__(self):
        if getattr(self, "_h", None):
            dlib().kiln_dit_destroy(self._h)
            self._h = None

    def set_step_weights(self, t_lin1, t_lin2, t_norm, final_mod1, final_mod2, x_embed, final_lin):
        D = self.D
        sizes = dict(t_lin1=D * D, t_lin2=3 * D * D, t_norm=D, final_mod1=256 * D, final_mod2=2 * D * 256,
                     x_embed=D * 68, final_lin=64 * D)
        args = dict(t_lin1=t_lin1, t_lin2=t_lin2, t_norm=t_norm, final_mod1=final_mod1, final_mod2=final_mod2,
                    x_embed=x_embed, final_lin=final_lin)
        w = StepWeightsC(*[_bf16(args[n], sizes[n], n) for n in _STEP_FIELDS])
        _check(dlib().kiln_dit_set_step_weights(self._h, ctypes.byref(w)))

    def set_block(self, i, sa_q, sa_k, sa_v, sa_o, ca_q, ca_o, ca_k, ca_v, mlp1, mlp2, sa_qn, sa_kn, ca_qn, ca_kn,
                  mod):
        """bf16 device weights [out, in]; mod: the six adaLN weights (sa1 [256, D], sa2 [3D, 256], ca1, ca2, mlp1,
        mlp2)."""
        D, F, C = self.D, self.F, self.ctx_dim
        v = dict(sa_q=sa_q, sa_k=sa_k, sa_v=sa_v, sa_o=sa_o, ca_q=ca_q, ca_o=ca_o, ca_k=ca_k, ca_v=ca_v, mlp1=mlp1,
                 mlp2=mlp2, sa_qn=sa_qn, sa_kn=sa_kn, ca_qn=ca_qn, ca_kn=ca_kn)
        n = dict(sa_q=D * D, sa_k=D * D, sa_v=D * D, sa_o=D * D, ca_q=D * D, ca_o=D * D, ca_k=D * C, ca_v=D * C,
                 mlp1=F * D, mlp2=D * F, sa_qn=128, sa_kn=128, ca_qn=128, ca_kn=128)
        for j, name in enumerate(["mod_sa1", "mod_sa2", "mod_ca1", "mod_ca2", "mod_mlp1", "mod_mlp2"]):
            v[name] = mod[j]
            n[name] = 256 * D if j % 2 == 0 else 3 * D * 256
        w = BlockWeights(*[_bf16(v[k], n[k], k) for k in _BLOCK_FIELDS])
        _check(dlib().kiln_dit_set_block(self._h, i, ctypes.byref(w)))

    def cache_context(self, ctx, real=None, length=None, fp32=False):
        """ctx [rows, ctx_dim] fp32 device; the first `real` rows are real, the context counts `length` rows
        (zero padding beyond real, default max(512, real) as the reference pads)."""
        real = ctx.shape[0] if real is None else real
        length = max(512, real) if length is None else length
        if ctx.shape[1] != self.ctx_dim or ctx.shape[0] < real:
            raise ValueError(f"context of shape {tuple(ctx.shape)}: need >= {real} rows of {self.ctx_dim}")
        h = _vp()
        _check(dlib().kiln_dit_cache_context(self._h, _f32(ctx, name="context"), real, length, int(fp32),
                                             ctypes.byref(h)))
        return Context(h, real, length)

    def forward(self, outs, latent, t, contexts, nag=None, cache=None, fp32=False):
        """Dit::forward_batch: outs / contexts lists of B (1..3); latent [16, Hl, Wl] fp32 device."""
        B = len(contexts)
        Hl, Wl = latent.shape[-2], latent.shape[-1]
        n = 16 * Hl * Wl
        po = (_vp * B)(*[_f32(o, n, "output").value for o in outs[:B]])
        pc = (_vp * B)(*[c.handle.value for c in contexts])
        _check(dlib().kiln_dit_forward(self._h, po, _f32(latent, n, "latent"), Hl, Wl, t, pc, B, _nag(nag),
                                       cache.handle if cache is not None else None, int(fp32)))
        return outs

    def step_tables(self, t):
        """The modulation vectors [blocks * 9D + 2D] for timestep t (Dit::step_tables)."""
        mods = torch.empty(self.blocks * 9 * self.D + 2 * self.D, device="cuda")
        _check(dlib().kiln_dit_step_tables(self._h, t, _p(mods)))
        return mods

    def run_block(self, i, X, mods, Hp, Wp, contexts, nag=None, fp32=False):
        """One block on X [B*T, D] (in place) with modulation mods [9D]."""
        B = len(contexts)
        pc = (_vp * B)(*[c.handle.value for c in contexts])
        _check(dlib().kiln_dit_run_block(self._h, i, _f32(X, B * Hp * Wp * self.D, "X"), _f32(mods, 9 * self.D, "mods"),
                                         Hp, Wp, pc, B, _nag(nag), int(fp32)))
        return X

    def sample(self, x, pos, neg=None, nag=None, nag_sigma_end=0.0, batch_cfg=True, fp32=False, init=None,
               mask=None, on_step=None, cancel=None, **params):
        """sample() (engine/src/pipeline.cu:415-598) with this model: x [16, Hl, Wl] fp32 (overwritten);
        params: the kiln_sample_params fields (steps, cfg, shift, denoise, seed, sampler, scheduler, ...).
        on_step(step, steps, sigma) after each step; cancel: a ctypes.c_int polled between steps. Returns the
        number of steps the step cache skipped."""
        from .sampler import make_params
        sp, keep = make_params(x, **params)
        Hl, Wl = x.shape[-2], x.shape[-1]
        n = 16 * Hl * Wl
        cb = STEP_FN(lambda u, s, k, sg, xp, vp, ms: on_step(s, k, sg)) if on_step else STEP_FN()
        skips = _i(0)
        _check(dlib().kiln_dit_sample(self._h, _f32(x, n, "x"), Hl, Wl, pos.handle, neg.handle if neg else None,
                                      _nag(nag), nag_sigma_end, int(batch_cfg), int(fp32), ctypes.byref(sp),
                                      _f32(init, n, "init") if init is not None else None,
                                      _f32(mask, Hl * Wl, "mask") if mask is not None else None, cb, None,
                                      ctypes.byref(cancel) if cancel is not None else None, ctypes.byref(skips)))
        del keep
        return skips.value
