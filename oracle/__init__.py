"""CPU oracle of the fused attention path — TEST INFRASTRUCTURE ONLY.

Loaded only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, always as the
checker (or the timed CPU baseline), never as a product path. numpy in, numpy out.
See oracle/oracle.c for the reference file:line each function restates and what pins it.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i = ctypes.c_int


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            from . import build as _b  # noqa: F401  (oracle/build.py)
            _b.build()
        L = ctypes.CDLL(path)
        L.oracle_ref_attn_f32.argtypes = [_f32p, _i, _f32p, _i, _f32p, _i, _f32p, _i, _i, _i, _i, _i, _i]
        L.oracle_attn_f64.argtypes = [_f32p, _i, _f32p, _i, _f32p, _i, _f32p, _i, _i, _i, _i, _i, _i, _i,
                                      ctypes.c_double]
        L.oracle_attn_f16sem.argtypes = [_f32p, _i, _f32p, _i, _f32p, _i, _f32p, _i, _i, _i, _i, _i, _i]
        L.oracle_rmsnorm_rows.argtypes = [_f32p, _f32p, ctypes.c_void_p, ctypes.c_long, _i, ctypes.c_float]
        L.oracle_layernorm_mod.argtypes = [_f32p, _f32p, _f32p, _f32p, ctypes.c_long, _i, ctypes.c_float]
        L.oracle_add_gated.argtypes = [_f32p, _f32p, ctypes.c_void_p, ctypes.c_long, _i]
        L.oracle_linear16.argtypes = [ctypes.c_void_p, ctypes.c_void_p, _i, _u16p, _i, _u16p, _i, _i, ctypes.c_void_p,
                                      ctypes.c_void_p, _i, _i, ctypes.c_void_p, ctypes.c_float]
        L.oracle_matvec_bf16.argtypes = [_f32p, _u16p, _f32p, ctypes.c_void_p, _i, _i]
        L.oracle_patchify.argtypes = [_f32p, _f32p, _i, _i]
        L.oracle_unpatchify.argtypes = [_f32p, _f32p, _i, _i]
        L.oracle_linear_f32.argtypes = [_f32p, _f32p, _u16p, _i, _i, _i]
        L.oracle_rope_half.argtypes = [_f32p, _i, _i, _i, _i, _f32p, _f32p]
        L.oracle_cosmos_rope.argtypes = [_f32p, _f32p, _i, _i]
        L.oracle_nag.argtypes = [_f32p, _i, _f32p, _i, _i, _i, ctypes.c_float, ctypes.c_float, ctypes.c_float]
        L.oracle_torch_randn.argtypes = [_f32p, ctypes.c_uint64, ctypes.c_size_t]
        L.oracle_torch_randn.restype = _i
        L.oracle_f32_to_f16.argtypes = [_u16p, _f32p, ctypes.c_size_t]
        L.oracle_f16_to_f32.argtypes = [_f32p, _u16p, ctypes.c_size_t]
        L.oracle_num_threads.restype = _i
        _LIB = L
    return _LIB


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def num_threads():
    return lib().oracle_num_threads()


def ref_attn_f32(q, k, v, H, Dh=128, npad=0):
    """Reference fp32 two-pass attention (bench/flash_test.cu:10-32). q [Tq, H*Dh], k/v [Tk, H*Dh]."""
    q, k, v = _c32(q), _c32(k), _c32(v)
    out = np.empty_like(q)
    lib().oracle_ref_attn_f32(out, q.shape[1], q, q.shape[1], k, k.shape[1], v, v.shape[1], q.shape[0], k.shape[0],
                              H, Dh, npad)
    return out


def attn_f64(q, k, v, H, Dh=128, npad=0, causal=False, scale=0.0):
    """Double-accumulation golden attention (optionally causal)."""
    q, k, v = _c32(q), _c32(k), _c32(v)
    out = np.empty((q.shape[0], H * Dh), np.float32)
    lib().oracle_attn_f64(out, out.shape[1], q, q.shape[1], k, k.shape[1], v, v.shape[1], q.shape[0], k.shape[0],
                          H, Dh, int(causal), npad, scale)
    return out


def attn_f16sem(q, k, v, H, npad=0, out16=True):
    """Emulation of the reference's fp16 tensor-core semantics (engine/src/tcflash.cuh)."""
    q, k, v = _c32(q), _c32(k), _c32(v)
    out = np.empty((q.shape[0], H * 128), np.float32)
    lib().oracle_attn_f16sem(out, out.shape[1], q, q.shape[1], k, k.shape[1], v, v.shape[1], q.shape[0], k.shape[0],
                             H, npad, int(out16))
    return out


def layernorm_mod(x, scale, shift, eps=1e-6):
    """Modulated LayerNorm over the rows of x [rows, dim] (engine/src/kernels.cu:678-697); new array."""
    x = _c32(x)
    y = np.empty_like(x)
    lib().oracle_layernorm_mod(y, x, _c32(scale), _c32(shift), x.shape[0], x.shape[1], eps)
    return y


def add_gated(x, y, gate=None):
    """x + gate * y per row (engine/src/kernels.cu:700-708); new array."""
    out = _c32(x).copy()
    y = _c32(y)
    g = _c32(gate) if gate is not None else None
    lib().oracle_add_gated(out, y, g.ctypes.data if g is not None else None, out.shape[0], out.shape[1])
    return out


EPI_F32, EPI_F16, EPI_GELU16, EPI_RESID = 0, 1, 2, 3


def linear16(x16, w16, epi=EPI_F32, y=None, gate=None, beta=0.0, a2=None, w2=None):
    """linear16 (engine/src/kernels.cu:573-609, epilogue tcgemm16.cuh:145-175) over fp16 bit patterns (uint16).

    x16 [T, cols], w16 [rows, cols], a2 [T, k2] / w2 [rows, k2] or None. F32/RESID: y is the fp32 [T, rows] input
    (zeros if None) and the result is a new fp32 array; F16/GELU16: returns fp16 bit patterns [T, rows]."""
    x16 = np.ascontiguousarray(x16, dtype=np.uint16)
    w16 = np.ascontiguousarray(w16, dtype=np.uint16)
    T, cols = x16.shape
    rows = w16.shape[0]
    k2 = 0
    if a2 is not None:
        a2 = np.ascontiguousarray(a2, dtype=np.uint16)
        w2 = np.ascontiguousarray(w2, dtype=np.uint16)
        k2 = a2.shape[1]
    if epi in (EPI_F32, EPI_RESID):
        out = _c32(y).copy() if y is not None else np.zeros((T, rows), np.float32)
        o32, o16 = out.ctypes.data, None
    else:
        out = np.zeros((T, rows), np.uint16)
        o32, o16 = None, out.ctypes.data
    g = _c32(gate) if gate is not None else None
    lib().oracle_linear16(o32, o16, rows, x16, T, w16, rows, cols, a2.ctypes.data if k2 else None,
                          w2.ctypes.data if k2 else None, k2, epi, g.ctypes.data if g is not None else None, beta)
    return out


def matvec_bf16(W, x, add=None):
    """y = W x (+ add), W bf16 bit patterns (uint16) [rows, cols] (engine/src/kernels.cu k_matvec)."""
    W = np.ascontiguousarray(W, dtype=np.uint16)
    y = np.empty(W.shape[0], np.float32)
    a = _c32(add) if add is not None else None
    lib().oracle_matvec_bf16(y, W, _c32(x), a.ctypes.data if a is not None else None, W.shape[0], W.shape[1])
    return y


def patchify(lat):
    """lat [16, Hl, Wl] -> tok [T, 68] (engine/src/dit.cu:174-182)."""
    lat = _c32(lat)
    Hl, Wl = lat.shape[1], lat.shape[2]
    tok = np.empty(((Hl // 2) * (Wl // 2), 68), np.float32)
    lib().oracle_patchify(tok, lat, Hl, Wl)
    return tok


def unpatchify(tok, Hl, Wl):
    """tok [T, 64] -> lat [16, Hl, Wl] (engine/src/dit.cu:184-191)."""
    lat = np.zeros((16, Hl, Wl), np.float32)
    lib().oracle_unpatchify(lat, _c32(tok), Hl, Wl)
    return lat


def linear_f32(x, W):
    """y = x W^T with W bf16 bit patterns [rows, cols] (engine/src/kernels.cu:508-529)."""
    x = _c32(x)
    W = np.ascontiguousarray(W, dtype=np.uint16)
    y = np.empty((x.shape[0], W.shape[0]), np.float32)
    lib().oracle_linear_f32(y, x, W, x.shape[0], W.shape[0], W.shape[1])
    return y


def rmsnorm_rows(x, w_bf16=None, eps=1e-6, dim=128):
    """Per-row RMSNorm over rows of `dim` (engine/src/kernels.cu:656-666); returns a new array."""
    x = _c32(x)
    y = np.empty_like(x)
    rows = x.size // dim
    wp = None
    if w_bf16 is not None:
        w_bf16 = np.ascontiguousarray(w_bf16, dtype=np.uint16)
        wp = w_bf16.ctypes.data
    lib().oracle_rmsnorm_rows(y, x, wp, rows, dim, eps)
    return y


def rope_half(x, H, cos_t, sin_t, Dh=128):
    """Rotate-half RoPE on x [T, ld] (engine/src/kernels.cu:759-772); returns a new array."""
    y = _c32(x).copy()
    T = y.shape[0]
    lib().oracle_rope_half(y, y.shape[1], T, H, Dh, _c32(cos_t), _c32(sin_t))
    return y


def cosmos_rope(Hp, Wp):
    """Cosmos 3D RoPE tables cos, sin [Hp*Wp, 64] (engine/src/dit.cu:196-215)."""
    c = np.empty((Hp * Wp, 64), np.float32)
    s = np.empty((Hp * Wp, 64), np.float32)
    lib().oracle_cosmos_rope(c, s, Hp, Wp)
    return c, s


def nag(a, an, s=5.0, tau=2.5, alpha=0.25):
    """NAG combine per row (engine/src/dit.cu:295-324); returns a new array."""
    y = _c32(a).copy()
    an = _c32(an)
    lib().oracle_nag(y, y.shape[1], an, an.shape[1], y.shape[0], y.shape[1], s, tau, alpha)
    return y


def torch_randn(seed, n):
    """Bit-exact torch.manual_seed(seed); torch.randn(n) (engine/src/pipeline.cu:17-64), n >= 16."""
    out = np.empty(n, np.float32)
    if lib().oracle_torch_randn(out, seed, n) != 0:
        raise ValueError("torch_randn restatement needs n >= 16")
    return out


def to_f16_bits(x):
    x = _c32(x)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_f32_to_f16(out.reshape(-1), x.reshape(-1), x.size)
    return out
