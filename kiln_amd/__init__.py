"""kiln_amd — MI355X (gfx950) fused attention path of Kiln's diffusion engine.

The product is the C-ABI library ``kiln_amd/libkiln_attn.so`` (declared in include/kiln_attn.h).
This module binds it with ctypes and offers thin torch-tensor wrappers named after the reference
op layer (engine/src/gpu.h:118-156): ``attention``, ``attention16``, ``rmsnorm``, ``rope_half``,
``nag_combine``, ``layernorm_mod``, ``add_gated``, ``linear16``, ``matvec``, ``silu``, ``gelu``, ``cfg_combine``
plus the batched/fused entry points. ``kiln_amd.dit`` and ``kiln_amd.sampler`` compose the DiT forward and
the flow-matching samplers from them. Tensors must live on the GPU; there is no CPU
fallback — when the library is missing, ``lib()`` raises.

Errors: a non-zero status from the library raises ``KilnError`` (the reference raises
std::runtime_error, engine/src/kernels.cu:870).
"""
import ctypes
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libkiln_attn.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "kiln_attn.h")

KILN_OK, KILN_EINVAL, KILN_EUNSUPPORTED, KILN_EHIP, KILN_ENOMEM = 0, 1, 2, 3, 4
KILN_F32, KILN_F16 = 0, 1
KILN_EPI_F32, KILN_EPI_F16, KILN_EPI_GELU16, KILN_EPI_RESID = 0, 1, 2, 3

_i, _ll, _f, _vp, _sz = ctypes.c_int, ctypes.c_longlong, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t

# symbol -> (restype, argtypes)
_SIGS = {
    "kiln_attn_status_string": (ctypes.c_char_p, [_i]),
    "kiln_attn_last_error": (ctypes.c_char_p, []),
    "kiln_attn_device_arch": (_i, [_i, ctypes.c_char_p, _i]),
    "kiln_attn_fwd_f32out": (_i, [_vp, _i, _vp, _i, _vp, _i, _vp, _i, _i, _i, _i, _i, _i, _i, _vp]),
    "kiln_attn_fwd_f16out": (_i, [_vp, _i, _vp, _i, _vp, _i, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "kiln_attn_fwd_exact": (_i, [_vp, _i, _vp, _i, _vp, _i, _vp, _i, _i, _i, _i, _i, _i, _i, _vp]),
    "kiln_rmsnorm_rows": (_i, [_vp, _vp, _vp, _i, _i, _f, _vp]),
    "kiln_rope_half": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp]),
    "kiln_layernorm_mod": (_i, [_vp, _vp, _vp, _vp, _i, _i, _f, _vp]),
    "kiln_layernorm_mod16": (_i, [_vp, _vp, _vp, _vp, _i, _i, _f, _vp]),
    "kiln_add_gated": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "kiln_linear16": (_i, [_vp, _i, _vp, _i, _vp, _i, _i, _i, _vp, _f, _vp, _vp, _i, _vp]),
    "kiln_matvec_bf16": (_i, [_vp, _vp, _vp, _vp, _i, _i, _vp]),
    "kiln_matvec_bf16_grouped": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "kiln_silu": (_i, [_vp, _vp, _sz, _vp]),
    "kiln_patchify": (_i, [_vp, _vp, _i, _i, _vp]),
    "kiln_unpatchify": (_i, [_vp, _vp, _i, _i, _i, _vp]),
    "kiln_linear_f32": (_i, [_vp, _i, _vp, _i, _vp, _i, _i, _i, _vp]),
    "kiln_cfg_combine": (_i, [_vp, _vp, _f, _sz, _vp]),
    "kiln_sub": (_i, [_vp, _vp, _vp, _sz, _vp]),
    "kiln_rel_l1": (_i, [_vp, _vp, _sz, _vp, _vp]),
    "kiln_torch_randn": (_i, [_vp, ctypes.c_uint64, _sz]),
    "kiln_flow_start": (_i, [_vp, _vp, _vp, _f, _sz, _vp]),
    "kiln_gelu": (_i, [_vp, _sz, _vp]),
    "kiln_flow_ersde_step": (_i, [_vp, _vp, _vp, _vp, _vp, _f, _f, _f, _f, _f, _f, _f, _i, _sz, _vp]),
    "kiln_flow_inpaint_in": (_i, [_vp, _vp, _vp, _vp, _vp, _f, _i, _vp]),
    "kiln_flow_denoised_masked": (_i, [_vp, _vp, _vp, _vp, _vp, _f, _i, _vp]),
    "kiln_flow_denoised": (_i, [_vp, _vp, _vp, _f, _sz, _vp]),
    "kiln_flow_update": (_i, [_vp, _vp, _vp, _f, _f, _f, _sz, _vp]),
    "kiln_flow_euler_step": (_i, [_vp, _vp, _f, _f, _sz, _vp]),
    "kiln_flow_euler_den": (_i, [_vp, _vp, _f, _f, _sz, _vp]),
    "kiln_pad_circular": (_i, [_vp, _vp, _i, _i, _i, _i, _vp]),
    "kiln_fill_uniform_bf16": (_i, [_vp, _sz, ctypes.c_uint64, _f, _f, _vp]),
    "kiln_crop": (_i, [_vp, _vp, _i, _i, _i, _i, _vp]),
    "kiln_attn_dropin_workspace_bytes": (_sz, [_i, _i, _i]),
    "kiln_attn_workspace_reserve": (_i, [_sz]),
    "kiln_attn_set_workspace": (_i, [_vp, _sz]),
    "kiln_attn_workspace_release": (_i, []),
    "kiln_prof_enable": (_i, [_i]),
    "kiln_prof_report": (_i, [ctypes.c_char_p, _sz]),
    "kiln_prof_category": (_i, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_i)]),
    "kiln_attn_fwd_f16out_noalloc": (_i, [_vp, _i, _vp, _i, _vp, _i, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "kiln_attn_noalloc_scratch_bytes": (_sz, []),
    "kiln_linear16_prepped": (_i, [_vp, _i, _vp, _i, _vp, _i, _i, _i, _vp, _f, _vp, _vp, _i, _vp]),
    "kiln_linear16_prepped_weight_bytes": (_sz, [_i, _i]),
    "kiln_linear16_prepare_weight": (_i, [_vp, _vp, _i, _i, _i, _vp]),
    "kiln_nag_combine": (_i, [_vp, _i, _vp, _i, _i, _i, _i, _f, _f, _f, _vp]),
    "kiln_cosmos_rope_tables": (_i, [_vp, _vp, _i, _i]),
    "kiln_kv_prepped_bytes": (_sz, [_i, _i]),
    "kiln_kv_prepare": (_i, [_vp, _vp, _i, _vp, _i, _i, _i, _i, _vp, _f, _vp, _vp, _vp]),
    "kiln_attn_fwd_prepped": (_i, [_vp, _i, _i, _vp, _i, _i, _vp, _f, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "kiln_attn_fwd_prepped_batch": (_i, [_vp, _i, _i, _ll, _vp, _i, _i, _ll, _vp, _f, _vp, _vp, _vp, _i, _i, _i, _i,
                                         _i, _vp]),
    "kiln_attn_fwd_f16in": (_i, [_vp, _i, _i, _ll, _vp, _i, _ll, _vp, _i, _ll, _vp, _i, _ll, _i, _i, _i, _i, _i,
                                 _vp, _sz, _vp]),
    "kiln_attn_fwd_f16in_workspace_bytes": (_sz, [_i, _i, _i]),
    "kiln_dit_self_attn_fused": (_i, [_vp, _i, _i, _vp, _vp, _vp, _i, _i, _vp, _vp, _f, _vp, _vp, _i, _i, _i, _vp,
                                      _sz, _vp]),
    "kiln_dit_self_attn_workspace_bytes": (_sz, [_i, _i, _i]),
    "kiln_dit_self_attn_x16": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp, _f, _vp, _vp, _i, _i, _i, _vp, _sz, _vp]),
    "kiln_dit_self_attn_x16_workspace_bytes": (_sz, [_i, _i, _i]),
    "kiln_dit_cross_attn_x16": (_i, [_vp, _vp, _i, _i, _vp, _vp, _vp, _f, _i, _i, _i, _vp, _vp, _vp, _vp, _i, _i, _f,
                                     _f, _f, _vp, _sz, _vp]),
    "kiln_cross_attn_nag": (_i, [_vp, _vp, _i, _i, _vp, _i, _i, _vp, _f, _i, _i, _i, _vp, _vp, _vp, _vp, _i, _i, _f,
                                 _f, _f, _vp]),
}

_LIB = None


class KilnError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"kiln status {status}: {msg}")
        self.status = status


def lib():
    """Load libkiln_attn.so (build it first with ``python -m kiln_amd.build``)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m kiln_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def prof_enable(on=True):
    """Starts (or stops) per-category GPU timing of the library's entry points (the reference's --profile)."""
    _check(lib().kiln_prof_enable(int(bool(on))))


def prof_report():
    """The per-category report of the current profile: {category: (ms, calls)} and its text form."""
    buf = ctypes.create_string_buffer(1 << 14)
    _check(lib().kiln_prof_report(buf, len(buf)))
    text = buf.value.decode()
    cats = {}
    for ln in text.splitlines():
        parts = ln.split()
        if len(parts) >= 3 and parts[0] != "sum":
            ms, calls = ctypes.c_double(), ctypes.c_int()
            _check(lib().kiln_prof_category(parts[0].encode(), ctypes.byref(ms), ctypes.byref(calls)))
            cats[parts[0]] = (ms.value, calls.value)
    return cats, text


def header_symbols(path=HEADER_PATH):
    """Function names declared in include/kiln_attn.h."""
    with open(path) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(kiln_[a-z_0-9]+)\s*\(", text, flags=re.M)))


def _check(rc):
    if rc != KILN_OK:
        msg = lib().kiln_attn_last_error().decode()
        raise KilnError(rc, msg)


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _dt(t):
    import torch
    if t.dtype == torch.float16:
        return KILN_F16
    if t.dtype == torch.float32:
        return KILN_F32
    raise TypeError(f"unsupported dtype {t.dtype}")


def _bf16_bits(w):
    """bf16 weight tensor (or None) -> pointer; torch.bfloat16 storage is the bf16 bit pattern."""
    import torch
    if w is None:
        return None
    if w.dtype != torch.bfloat16 or not w.is_contiguous() or w.numel() < 128:
        raise TypeError("norm weights must be a contiguous bf16 tensor of >= 128 elements")
    return _ptr(w)


def _f32s(n, *ts):
    """Every tensor in ts (None skipped) is float32, contiguous, on one device and holds n elements; the kernels
    index n elements of each, so a mismatch would read or write out of bounds."""
    import torch
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"expected a contiguous float32 tensor, got {t.dtype} (contiguous={t.is_contiguous()})")
        if t.numel() != n:
            raise ValueError(f"expected {n} elements, got {t.numel()} (shape {tuple(t.shape)})")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")


def _ld(t):
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError("expected a 2-D row-major tensor")
    return t.stride(0)


# ---------------------------------------------------------------------------------------------
# reference-named op layer (engine/src/gpu.h)
# ---------------------------------------------------------------------------------------------
def attention(out, q, k, v, Tq, Tk, H, Dh=128, causal=False, npad=0, stream=None):
    """attention() (engine/src/gpu.h:149-153): fp32 q/k/v/out rows, head h at column h*Dh."""
    _check(lib().kiln_attn_fwd_f32out(_ptr(out), _ld(out), _ptr(q), _ld(q), _ptr(k), _ld(k), _ptr(v), _ld(v), Tq, Tk,
                                      H, Dh, int(causal), npad, _stream(stream)))
    return out


def attention16(out, q, k, v, Tq, Tk, H, Dh=128, npad=0, stream=None):
    """attention16() (engine/src/gpu.h:155-156): fp32 q/k/v, fp16 out."""
    _check(lib().kiln_attn_fwd_f16out(_ptr(out), _ld(out), _ptr(q), _ld(q), _ptr(k), _ld(k), _ptr(v), _ld(v), Tq, Tk,
                                      H, Dh, npad, _stream(stream)))
    return out


def attention_exact(out, q, k, v, Tq, Tk, H, Dh, causal=False, npad=0, stream=None):
    """Exact fp32 attention (the reference's --fp32 fallback semantics)."""
    _check(lib().kiln_attn_fwd_exact(_ptr(out), _ld(out), _ptr(q), _ld(q), _ptr(k), _ld(k), _ptr(v), _ld(v), Tq, Tk,
                                     H, Dh, int(causal), npad, _stream(stream)))
    return out


def rmsnorm(y, x, w=None, rows=None, dim=128, eps=1e-6, stream=None):
    """rmsnorm() over rows of `dim` (engine/src/gpu.h:133); fp32, in place allowed."""
    rows = x.numel() // dim if rows is None else rows
    _check(lib().kiln_rmsnorm_rows(_ptr(y), _ptr(x), _bf16_bits(w), rows, dim, eps, _stream(stream)))
    return y


def rope_half(x, T, H, Dh, cos_t, sin_t, stream=None):
    """rope_half() (engine/src/gpu.h:145): in place on dense fp32 rows [T, H*Dh]."""
    _check(lib().kiln_rope_half(_ptr(x), T, H, Dh, _ptr(cos_t), _ptr(sin_t), _stream(stream)))
    return x


def layernorm_mod(y, x, scale, shift, eps=1e-6, stream=None):
    """Modulated LayerNorm of the DiT block (engine/src/kernels.cu:678-697): x [rows, dim] fp32, y fp32 or fp16."""
    import torch
    rows, dim = x.shape
    fn = lib().kiln_layernorm_mod16 if y.dtype == torch.float16 else lib().kiln_layernorm_mod
    _check(fn(_ptr(y), _ptr(x), _ptr(scale), _ptr(shift), rows, dim, eps, _stream(stream)))
    return y


def add_gated(x, y, gate=None, stream=None):
    """Gated residual x += gate * y (engine/src/kernels.cu:700-708); x, y [rows, dim] fp32."""
    rows, dim = x.shape
    _check(lib().kiln_add_gated(_ptr(x), _ptr(y), _ptr(gate), rows, dim, _stream(stream)))
    return x


def nag_combine(a, an, scale=5.0, tau=2.5, alpha=0.25, stream=None):
    """k_nag (engine/src/dit.cu:295-324): a <- NAG(a, an) in place, rows of a.shape[1]."""
    _check(lib().kiln_nag_combine(_ptr(a), _ld(a), _ptr(an), _ld(an), _dt(a), a.shape[0], a.shape[1], scale, tau,
                                  alpha, _stream(stream)))
    return a


def cosmos_rope_tables(Hp, Wp):
    """Cosmos 3D RoPE cos/sin tables [Hp*Wp, 64] as CPU float32 tensors (engine/src/dit.cu:196-215)."""
    import torch
    c = torch.empty(Hp * Wp, 64, dtype=torch.float32)
    s = torch.empty(Hp * Wp, 64, dtype=torch.float32)
    _check(lib().kiln_cosmos_rope_tables(_ptr(c), _ptr(s), Hp, Wp))
    return c, s


# ---------------------------------------------------------------------------------------------
# MI355X-native batched / fused entry points
# ---------------------------------------------------------------------------------------------
def kv_prepped_bytes(Tk, H):
    return lib().kiln_kv_prepped_bytes(Tk, H)


def kv_prepare(k, v, H, k_norm_w=None, eps=1e-6, rope=None, stream=None):
    """Prepare K/V (fp16 tiled MFMA order, optional K RMSNorm/RoPE); returns a uint8 device buffer."""
    import torch
    Tk = k.shape[0]
    buf = torch.empty(max(kv_prepped_bytes(Tk, H), 16), dtype=torch.uint8, device=k.device)
    rc, rs = rope if rope is not None else (None, None)
    _check(lib().kiln_kv_prepare(_ptr(buf), _ptr(k), _ld(k), _ptr(v), _ld(v), _dt(k), Tk, H, _bf16_bits(k_norm_w),
                                 eps, _ptr(rc), _ptr(rs), _stream(stream)))
    return buf


def attn_prepped(out, q, kvp, Tk, H, npad=0, q_norm_w=None, eps=1e-6, rope=None, stream=None):
    rc, rs = rope if rope is not None else (None, None)
    _check(lib().kiln_attn_fwd_prepped(_ptr(out), _dt(out), _ld(out), _ptr(q), _dt(q), _ld(q), _bf16_bits(q_norm_w),
                                       eps, _ptr(rc), _ptr(rs), _ptr(kvp), q.shape[0], Tk, H, npad, _stream(stream)))
    return out


def attn_prepped_batch(out, q, kvps, Tq, Tk, H, npad=0, q_norm_w=None, eps=1e-6, rope=None, stream=None):
    """B query sets (rows b*Tq of q/out) against prepared K/V buffers kvps[b], one launch."""
    B = len(kvps)
    rc, rs = rope if rope is not None else (None, None)
    ptrs = (ctypes.c_void_p * B)(*[k.data_ptr() for k in kvps])
    _check(lib().kiln_attn_fwd_prepped_batch(_ptr(out), _dt(out), _ld(out), Tq * _ld(out), _ptr(q), _dt(q), _ld(q),
                                             Tq * _ld(q), _bf16_bits(q_norm_w), eps, _ptr(rc), _ptr(rs),
                                             ctypes.cast(ptrs, _vp), B, Tq, Tk, H, npad, _stream(stream)))
    return out


def attn_f16in(out, q, k, v, B, Tq, Tk, H, npad=0, workspace=None, stream=None):
    """Batched fp16 attention: q/k/v/out are [B*T, ld] with batch b at rows b*T."""
    ws = _ptr(workspace) if workspace is not None else None
    wsb = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _check(lib().kiln_attn_fwd_f16in(_ptr(out), _dt(out), _ld(out), Tq * _ld(out), _ptr(q), _ld(q), Tq * _ld(q),
                                     _ptr(k), _ld(k), Tk * _ld(k), _ptr(v), _ld(v), Tk * _ld(v), B, Tq, Tk, H, npad,
                                     ws, wsb, _stream(stream)))
    return out


def dit_self_attn_workspace_bytes(B, T, H):
    return lib().kiln_dit_self_attn_workspace_bytes(B, T, H)


def dit_self_attn(out, q, k, v, B, T, H, q_norm_w, k_norm_w, rope, eps=1e-6, workspace=None, stream=None):
    """Fused DiT self-attention (QK-RMSNorm + RoPE + attention) of a CFG batch; q/k/v [B*T, ld]."""
    if not (_ld(q) == _ld(k) == _ld(v)):
        raise ValueError("q, k, v must share one row stride")
    ws = _ptr(workspace) if workspace is not None else None
    wsb = workspace.numel() * workspace.element_size() if workspace is not None else 0
    rc, rs = rope
    _check(lib().kiln_dit_self_attn_fused(_ptr(out), _dt(out), _ld(out), _ptr(q), _ptr(k), _ptr(v), _dt(q), _ld(q),
                                          _bf16_bits(q_norm_w), _bf16_bits(k_norm_w), eps, _ptr(rc), _ptr(rs), B, T,
                                          H, ws, wsb, _stream(stream)))
    return out


def cross_attn_nag(out, q, B, T, H, kvps, Lks, npads, q_norm_w=None, eps=1e-6, kvp_neg=None, Lk_neg=0, npad_neg=0,
                   out_neg=None, scale=5.0, tau=2.5, alpha=0.25, stream=None):
    """DiT cross-attention of a CFG batch with optional NAG on item 0 (engine/src/dit.cu:473-487)."""
    n = len(kvps)
    ptrs = (ctypes.c_void_p * n)(*[k.data_ptr() for k in kvps])
    lks = (ctypes.c_int * n)(*Lks)
    nps = (ctypes.c_int * n)(*npads)
    _check(lib().kiln_cross_attn_nag(_ptr(out), _ptr(out_neg), _dt(out), _ld(out), _ptr(q), _dt(q), _ld(q),
                                     _bf16_bits(q_norm_w), eps, B, T, H, ctypes.cast(ptrs, _vp),
                                     ctypes.cast(lks, _vp), ctypes.cast(nps, _vp), _ptr(kvp_neg), Lk_neg, npad_neg,
                                     scale, tau, alpha, _stream(stream)))
    return out


def linear16_prepare_weight(w, stream=None):
    """weight_to_f16 for a linear16 weight (engine/src/kernels.cu:531-544) into the prepared layout.

    w: fp16 or bf16 [rows, cols] (contiguous). Returns a PreppedWeight for linear16(..., w16=<it>)."""
    import torch
    if not w.is_contiguous():
        raise ValueError("linear16_prepare_weight: w must be contiguous")
    rows, cols = w.shape
    nbytes = lib().kiln_linear16_prepped_weight_bytes(rows, cols)
    buf = torch.empty(max(nbytes, 2) // 2, dtype=torch.float16, device=w.device)
    _check(lib().kiln_linear16_prepare_weight(_ptr(buf), _ptr(w), rows, cols, int(w.dtype == torch.bfloat16),
                                              _stream(stream)))
    return PreppedWeight(buf, rows, cols)


class PreppedWeight:
    """A linear16 weight in the prepared tile layout (kiln_linear16_prepare_weight)."""

    def __init__(self, buf, rows, cols):
        self.buf, self.shape = buf, (rows, cols)

    def is_contiguous(self):
        return True


def linear16(y, x16, w16, epi=KILN_EPI_F32, gate=None, beta=0.0, a2=None, w2=None, stream=None):
    """linear16() (engine/src/kernels.cu:573-609): acc = x16 w16^T (+ a2 w2^T) with epilogue `epi`.

    x16 fp16 [T, cols], w16 fp16 [rows, cols] or a PreppedWeight, y [T, >= rows] (fp32 for F32/RESID, fp16 for F16/GELU16,
    row stride y.stride(0)); a2 [T, k2] / w2 [rows, k2] fp16 or None."""
    T, cols = x16.shape
    rows = w16.shape[0]
    k2 = 0 if a2 is None else a2.shape[1]
    for t in (x16, w16, a2, w2):
        if t is not None and not t.is_contiguous():
            raise ValueError("linear16: x16, w16, a2 and w2 must be dense (contiguous) rows")
    if y.stride(1) != 1:
        raise ValueError("linear16: y rows must be contiguous")
    if isinstance(w16, PreppedWeight):
        fn, wptr = lib().kiln_linear16_prepped, _ptr(w16.buf)
    else:
        fn, wptr = lib().kiln_linear16, _ptr(w16)
    _check(fn(_ptr(y), y.stride(0), _ptr(x16), T, wptr, rows, cols, epi, _ptr(gate), beta, _ptr(a2), _ptr(w2), k2,
              _stream(stream)))
    return y


def matvec(y, w_bf16, x, add=None, stream=None):
    """matvec (engine/src/gpu.h:122): y = W x (+ add), W bf16 [rows, cols]."""
    _check(lib().kiln_matvec_bf16(_ptr(y), _ptr(w_bf16), _ptr(x), _ptr(add), w_bf16.shape[0], w_bf16.shape[1],
                                  _stream(stream)))
    return y


def matvec_grouped(y, w_bf16, x, add=None, stream=None):
    """groups matvecs in one launch: w_bf16 [groups, rows, cols], x [groups, cols], y [groups, rows], add [rows]."""
    G, rows, cols = w_bf16.shape
    _check(lib().kiln_matvec_bf16_grouped(_ptr(y), _ptr(w_bf16), _ptr(x), _ptr(add), G, rows, cols, _stream(stream)))
    return y


def silu(y, x, stream=None):
    """silu (engine/src/kernels.cu:735-739), elementwise over x.numel()."""
    _check(lib().kiln_silu(_ptr(y), _ptr(x), x.numel(), _stream(stream)))
    return y


def patchify(tok, latent, stream=None):
    """k_patchify (engine/src/dit.cu:174-182): latent [16, Hl, Wl] -> tok [T, 68]."""
    _check(lib().kiln_patchify(_ptr(tok), _ptr(latent), latent.shape[1], latent.shape[2], _stream(stream)))
    return tok


def unpatchify(latent, tok, stream=None):
    """k_unpatchify (engine/src/dit.cu:184-191): tok [T, >= 64] (row stride tok.stride(0)) -> latent [16, Hl, Wl]."""
    _check(lib().kiln_unpatchify(_ptr(latent), _ptr(tok), tok.stride(0), latent.shape[1], latent.shape[2],
                                 _stream(stream)))
    return latent


def linear_f32(y, x, w_bf16, stream=None):
    """linear (engine/src/kernels.cu:508-529) for small fp32 layers: y [T, rows] = x [T, cols] W^T, W bf16."""
    _check(lib().kiln_linear_f32(_ptr(y), y.stride(0), _ptr(x), x.stride(0), _ptr(w_bf16), x.shape[0],
                                 w_bf16.shape[0], w_bf16.shape[1], _stream(stream)))
    return y


def cfg_combine(v, vn, cfg, stream=None):
    """cfg_combine (engine/src/kernels.cu:1058-1062): v = vn + cfg (v - vn)."""
    _f32s(v.numel(), v, vn)
    _check(lib().kiln_cfg_combine(_ptr(v), _ptr(vn), cfg, v.numel(), _stream(stream)))
    return v


def flow_start(x, noise, sigma, init=None, stream=None):
    """k_start (engine/src/pipeline.cu:304-307): x = sigma noise + (1 - sigma) init."""
    _f32s(x.numel(), x, noise, init)
    _check(lib().kiln_flow_start(_ptr(x), _ptr(noise), _ptr(init), sigma, x.numel(), _stream(stream)))
    return x


def flow_euler_step(x, v, sigma, sigma_next, stream=None):
    """k_denoised + k_euler_step (engine/src/pipeline.cu:318-331) without a mask, in place on x."""
    _f32s(x.numel(), x, v)
    _check(lib().kiln_flow_euler_step(_ptr(x), _ptr(v), sigma, sigma_next, x.numel(), _stream(stream)))
    return x


def flow_euler_den(x, den, sigma, sigma_next, stream=None):
    """k_euler_step (engine/src/pipeline.cu:326-331) on a given denoised estimate (the masked path):
    x = x + (x - den) / sigma * (sigma_next - sigma), in place."""
    _f32s(x.numel(), x, den)
    _check(lib().kiln_flow_euler_den(_ptr(x), _ptr(den), sigma, sigma_next, x.numel(), _stream(stream)))
    return x


def sub(y, a, b, stream=None):
    """k_sub (engine/src/dit.cu:337-340): y = a - b."""
    _f32s(a.numel(), y, a, b)
    _check(lib().kiln_sub(_ptr(y), _ptr(a), _ptr(b), a.numel(), _stream(stream)))
    return y


def rel_l1(a, b, acc, stream=None):
    """k_rel_l1 (engine/src/dit.cu:327-335): acc[0] = sum|a - b|, acc[1] = sum|b| (device float[2])."""
    _check(lib().kiln_rel_l1(_ptr(a), _ptr(b), a.numel(), _ptr(acc), _stream(stream)))
    return acc


def dit_self_attn_x16(out, x16, wqkv, B, T, H, q_norm_w, k_norm_w, rope, eps=1e-6, workspace=None, stream=None):
    """The DiT self-attention section from the fp16 LayerNorm output: QKV projection (wqkv: a PreppedWeight of
    [3D, D]) with QK-norm + RoPE + K/V preparation fused into its epilogue, then attention (kiln_dit_self_attn_x16)."""
    import torch
    if workspace is None:
        workspace = torch.empty(lib().kiln_dit_self_attn_x16_workspace_bytes(B, T, H), dtype=torch.uint8,
                                device=x16.device)
    rc, rs = rope
    _check(lib().kiln_dit_self_attn_x16(_ptr(out), _dt(out), _ld(out), _ptr(x16), _ptr(wqkv.buf),
                                        _bf16_bits(q_norm_w), _bf16_bits(k_norm_w), eps, _ptr(rc), _ptr(rs), B, T, H,
                                        _ptr(workspace), workspace.numel(), _stream(stream)))
    return out


def torch_randn(seed, n):
    """torch_randn (engine/src/pipeline.cu:17-64): torch.manual_seed(seed); torch.randn(n) on the host, as a CPU
    float32 tensor (the library's own MT19937 + Box-Muller)."""
    import torch
    out = torch.empty(n, dtype=torch.float32)
    _check(lib().kiln_torch_randn(_ptr(out), seed, n))
    return out


def dit_cross_attn_x16(out, x16, wq, B, T, H, kvps, Lks, npads, q_norm_w, eps=1e-6, kvp_neg=None, Lk_neg=0,
                       npad_neg=0, out_neg=None, scale=5.0, tau=2.5, alpha=0.25, workspace=None, stream=None):
    """The DiT cross-attention section from the fp16 LayerNorm output: cross-Q projection (wq: a PreppedWeight)
    with the Q RMSNorm in its epilogue, then cross-attention + NAG (kiln_dit_cross_attn_x16)."""
    import torch
    D = H * 128
    if workspace is None:
        workspace = torch.empty(B * T * D * 2, dtype=torch.uint8, device=x16.device)
    n = len(kvps)
    ptrs = (ctypes.c_void_p * n)(*[k.data_ptr() for k in kvps])
    lks = (ctypes.c_int * n)(*Lks)
    nps = (ctypes.c_int * n)(*npads)
    _check(lib().kiln_dit_cross_attn_x16(_ptr(out), _ptr(out_neg), _dt(out), _ld(out), _ptr(x16), _ptr(wq.buf),
                                         _bf16_bits(q_norm_w), eps, B, T, H, ctypes.cast(ptrs, _vp),
                                         ctypes.cast(lks, _vp), ctypes.cast(nps, _vp), _ptr(kvp_neg), Lk_neg, npad_neg,
                                         scale, tau, alpha, _ptr(workspace), workspace.numel(), _stream(stream)))
    return out


def flow_denoised(den, x, v, sigma, stream=None):
    """k_denoised without a mask (engine/src/pipeline.cu:318-324): den = x - v sigma."""
    _f32s(x.numel(), den, x, v)
    _check(lib().kiln_flow_denoised(_ptr(den), _ptr(x), _ptr(v), sigma, x.numel(), _stream(stream)))
    return den


def flow_update(x, den, a, b, old=None, c=0.0, stream=None):
    """k_update (engine/src/pipeline.cu:333-337): x = a x + b den + c old."""
    _f32s(x.numel(), x, den, old)
    _check(lib().kiln_flow_update(_ptr(x), _ptr(den), _ptr(old), a, b, c, x.numel(), _stream(stream)))
    return x


def flow_inpaint_in(xin, x, noise, init, mask, sigma, stream=None):
    """k_inpaint_in (engine/src/pipeline.cu:309-315): latents [16, ...], mask [P] per pixel."""
    _f32s(mask.numel(), mask)
    _f32s(16 * mask.numel(), xin, x, noise, init)
    _check(lib().kiln_flow_inpaint_in(_ptr(xin), _ptr(x), _ptr(noise), _ptr(init), _ptr(mask), sigma, mask.numel(),
                                      _stream(stream)))
    return xin


def flow_denoised_masked(den, xin, v, init, mask, sigma, stream=None):
    """k_denoised with a mask (engine/src/pipeline.cu:317-324): pinned to init where the mask is 0."""
    _f32s(mask.numel(), mask)
    _f32s(16 * mask.numel(), den, xin, v, init)
    _check(lib().kiln_flow_denoised_masked(_ptr(den), _ptr(xin), _ptr(v), _ptr(init), _ptr(mask), sigma, mask.numel(),
                                           _stream(stream)))
    return den


def gelu(x, stream=None):
    """gelu (engine/src/kernels.cu:728-733): in place, fp32, erf form."""
    _f32s(x.numel(), x)
    _check(lib().kiln_gelu(_ptr(x), x.numel(), _stream(stream)))
    return x


def flow_ersde_step(x, den, old, oldd, noise, c, stream=None):
    """k_ersde (engine/src/pipeline.cu:345-359) with the coefficients c = (a, b, c2, inv2, c3, inv3, cn, stage)."""
    a, b, c2, inv2, c3, inv3, cn, stage = c
    _f32s(x.numel(), x, den, old, oldd, noise)
    _check(lib().kiln_flow_ersde_step(_ptr(x), _ptr(den), _ptr(old), _ptr(oldd), _ptr(noise), a, b, c2, inv2, c3, inv3,
                                      cn, stage, x.numel(), _stream(stream)))
    return x
