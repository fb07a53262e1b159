"""GPU parity of the HIP attention path against the CPU oracle (double-accumulation softmax attention).

Tolerance: max-abs <= 2e-3 and mean-abs <= 2e-4 against the fp32 reference,
on identical seeded inputs. Cases follow the reference harnesses (bench/tfa_test.cu:69-76 shapes,
Q,K ~ N(0, 1.5), V ~ N(0, 1)) and the BASELINE configs 1-4.
"""
import numpy as np
import pytest
import torch

import kiln_amd
import oracle
from tests.helpers import assert_close, errors, f16_round, randn

pytestmark = pytest.mark.gpu
H, D = 16, 128
DEV = "cuda:0"


def emulator_bar(emu, ref):
    """Bar for stress inputs outside the BASELINE configs (peaky softmax): the error that the reference's
    fp16 semantics (oracle.attn_f16sem) itself has on the same inputs, plus one fp16 ulp of the largest
    output for max-abs (the kernel and the emulator may round an output to neighbouring fp16 values),
    1.25x for mean-abs; never below the BASELINE bar."""
    emx, emn, _ = errors(emu, ref)
    top = float(np.abs(ref).max())
    ulp = 2.0 ** (np.floor(np.log2(max(top, 2.0 ** -14))) - 10)
    return dict(max_abs=max(2e-3, emx + ulp), mean_abs=max(2e-4, 1.25 * emn))


def _qkv(seed, Tq, Tk, scale_qk=1.5):
    q = randn(seed, Tq, H * D, scale=scale_qk)
    k = randn(seed + 1, Tk, H * D, scale=scale_qk)
    v = randn(seed + 2, Tk, H * D)
    return q, k, v


# ---- config 1: plain self-attention, fp16 Q/K/V ~ N(0,1) from torch_randn(0, 3*1536*2048) ----
def test_cfg1_plain_self_attention_f16(gpu):
    S = 1536
    x = randn(0, 3 * S * H * D)
    q, k, v = (f16_round(t.reshape(S, H * D)) for t in x.split(S * H * D))
    ref = oracle.attn_f64(q.numpy(), k.numpy(), v.numpy(), H)
    for od in (torch.float16, torch.float32):
        out = torch.empty(S, H * D, dtype=od, device=DEV)
        kiln_amd.attn_f16in(out, q.half().to(DEV), k.half().to(DEV), v.half().to(DEV), 1, S, S, H)
        torch.cuda.synchronize()
        assert_close(out.float().cpu().numpy(), ref, f"cfg1 S=1536 out={od}")


# ---- drop-ins: the reference harness shapes (bench/tfa_test.cu:69-76) through attention16/attention ----
TFA_SHAPES = [(1536, 1536, 0), (1536, 26, 486), (1000, 1000, 0), (1000, 77, 0), (3952, 3952, 0)]


@pytest.mark.parametrize("Tq,Tk,npad", TFA_SHAPES)
def test_dropin_attention16_tfa_shapes(gpu, Tq, Tk, npad):
    """The reference harness draws Q,K ~ N(0, 1.5) (bench/tfa_test.cu:39-42): scores have std 2.25, so
    the fp16 rounding of Q and K alone (the CUDA path's semantics) moves outputs by ~2e-3. These shapes
    are not BASELINE configs; the bar here is the reference's own: the error of the fp16-semantics
    emulator on the same inputs (x1.25), and rel_l2 at the published 6.9e-4 (README.md:570)."""
    q, k, v = _qkv(3, Tq, Tk)
    rows = np.random.default_rng(Tq).choice(Tq, size=min(Tq, 512), replace=False)
    qn, kn, vn = q.numpy()[rows], k.numpy(), v.numpy()
    ref = oracle.attn_f64(qn, kn, vn, H, npad=npad)
    emu32 = oracle.attn_f16sem(qn, kn, vn, H, npad=npad, out16=False)
    emu16 = oracle.attn_f16sem(qn, kn, vn, H, npad=npad, out16=True)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    out16 = torch.empty(Tq, H * D, dtype=torch.float16, device=DEV)
    kiln_amd.attention16(out16, qd, kd, vd, Tq, Tk, H, D, npad=npad)
    out32 = torch.empty(Tq, H * D, dtype=torch.float32, device=DEV)
    kiln_amd.attention(out32, qd, kd, vd, Tq, Tk, H, D, causal=False, npad=npad)
    torch.cuda.synchronize()
    for name, got, emu in (("attention16", out16.float().cpu().numpy()[rows], emu16),
                           ("attention", out32.cpu().numpy()[rows], emu32)):
        emx, emn, erl = errors(emu, ref)
        assert_close(got, ref, f"{name} {Tq}x{Tk}+{npad} (emulator max {emx:.2e} mean {emn:.2e} rel {erl:.2e})",
                     max_abs=max(2e-3, 1.25 * emx), mean_abs=max(2e-4, 1.25 * emn))
        assert errors(got, ref)[2] <= max(6.9e-4, 1.25 * erl)


def test_dropin_matches_fp16_semantics_emulator(gpu):
    """Per element, the kernel must sit at the fp16-semantics emulator, far inside the fp32 bar."""
    Tq, Tk = 256, 333
    q, k, v = _qkv(11, Tq, Tk)
    emu = oracle.attn_f16sem(q.numpy(), k.numpy(), v.numpy(), H, out16=False)
    ref = oracle.attn_f64(q.numpy(), k.numpy(), v.numpy(), H)
    out = torch.empty(Tq, H * D, dtype=torch.float32, device=DEV)
    kiln_amd.attention(out, q.to(DEV), k.to(DEV), v.to(DEV), Tq, Tk, H, D)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    mx_e, mn_e, _ = errors(got, emu)
    mx_r, mn_r, _ = errors(emu, ref)
    print(f"[parity] kernel vs emulator max {mx_e:.2e} mean {mn_e:.2e}; emulator vs f64 max {mx_r:.2e} mean {mn_r:.2e}")
    # the kernel must sit closer to the reference's fp16 semantics than those semantics sit to exact math
    assert mn_e <= mn_r, "kernel deviates from the fp16 semantics more than fp16 itself deviates from fp32"
    assert mx_e <= mx_r


# ---- configs 2 and 4: fused DiT self-attention (QK-RMSNorm + 3D RoPE), CFG batch 2 ----
def _dit_inputs(seed, T, B, wlow=None, dtype=torch.float16):
    """Q/K/V = X W^T with X ~ N(0,1) [B*T, 2048], W ~ U(+-1/sqrt(2048)) (torch Linear init)."""
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(B * T, H * D, generator=g)
    outs = []
    for i in range(3):
        W = (torch.rand(H * D, H * D, generator=g) * 2 - 1) / np.sqrt(H * D)
        outs.append((X @ W.T).to(dtype))
    if wlow is None:
        qw = torch.ones(D, dtype=torch.bfloat16)
        kw = torch.ones(D, dtype=torch.bfloat16)
    else:
        qw = (torch.rand(D, generator=g) * 2 + 1).to(torch.bfloat16)
        kw = (torch.rand(D, generator=g) * 2 + 1).to(torch.bfloat16)
    return outs, qw, kw


def _dit_reference(q, k, v, qw, kw, cos, sin, B, T, rows):
    """oracle: rmsnorm(Q), rmsnorm(K) per head, rope both, attention (engine/src/dit.cu:464-470)."""
    outs = []
    qwb = qw.view(torch.int16).numpy().view(np.uint16)
    kwb = kw.view(torch.int16).numpy().view(np.uint16)
    for b in range(B):
        qb = q[b * T:(b + 1) * T].float().numpy()
        kb = k[b * T:(b + 1) * T].float().numpy()
        vb = v[b * T:(b + 1) * T].float().numpy()
        qn = oracle.rope_half(oracle.rmsnorm_rows(qb, qwb).reshape(T, H * D), H, cos, sin)
        kn = oracle.rope_half(oracle.rmsnorm_rows(kb, kwb).reshape(T, H * D), H, cos, sin)
        outs.append((oracle.attn_f64(qn[rows], kn, vb, H), (qn[rows], kn, vb)))
    return outs


@pytest.mark.parametrize("Hp,Wp,wvar", [(32, 48, None), (32, 48, "u13"), (64, 64, None)])
def test_dit_self_attention_fused(gpu, Hp, Wp, wvar):
    T, B = Hp * Wp, 2
    (q, k, v), qw, kw = _dit_inputs(5, T, B, wvar)
    cos, sin = oracle.cosmos_rope(Hp, Wp)
    rows = np.sort(np.random.default_rng(T).choice(T, size=min(T, 384), replace=False))
    refs = _dit_reference(q, k, v, qw, kw, cos, sin, B, T, rows)
    out = torch.empty(B * T, H * D, dtype=torch.float16, device=DEV)
    rope = (torch.from_numpy(cos).to(DEV), torch.from_numpy(sin).to(DEV))
    kiln_amd.dit_self_attn(out, q.to(DEV), k.to(DEV), v.to(DEV), B, T, H, qw.to(DEV), kw.to(DEV), rope)
    torch.cuda.synchronize()
    o = out.float().cpu().numpy()
    for b in range(B):
        ref, normed = refs[b]
        # norm weights 1 (torch RMSNorm init) = the BASELINE configs 2/4: strict bar; U(1,3): stress
        bar = {} if wvar is None else emulator_bar(oracle.attn_f16sem(*normed, H), ref)
        assert_close(o[b * T:(b + 1) * T][rows], ref, f"DiT self T={T} b={b} w={wvar}", **bar)


def test_dit_self_attention_fp32_inputs(gpu):
    """The reference's own DiT path hands fp32 Q/K/V to attention (engine/src/dit.cu:501-506)."""
    Hp, Wp, B = 16, 24, 2
    T = Hp * Wp
    (q, k, v), qw, kw = _dit_inputs(9, T, B, None, dtype=torch.float32)
    cos, sin = oracle.cosmos_rope(Hp, Wp)
    rows = np.arange(T)
    refs = _dit_reference(q, k, v, qw, kw, cos, sin, B, T, rows)
    out = torch.empty(B * T, H * D, dtype=torch.float32, device=DEV)
    rope = (torch.from_numpy(cos).to(DEV), torch.from_numpy(sin).to(DEV))
    kiln_amd.dit_self_attn(out, q.to(DEV), k.to(DEV), v.to(DEV), B, T, H, qw.to(DEV), kw.to(DEV), rope)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    for b in range(B):
        assert_close(o[b * T:(b + 1) * T], refs[b][0], f"DiT self fp32-in T={T} b={b}")


# ---- config 3: cross-attention over 512 context tokens, positive + negative, NAG ----
@pytest.mark.parametrize("L,npad,wvar", [(512, 0, None), (26, 486, None), (512, 0, "u13")])
def test_cross_attention_nag(gpu, L, npad, wvar):
    T, B = 1536, 2
    g = torch.Generator().manual_seed(21)
    qraw = (torch.randn(B * T, H * D, generator=g)).half()
    qw = torch.ones(D, dtype=torch.bfloat16) if wvar is None else (torch.rand(D, generator=g) * 2 + 1).to(torch.bfloat16)
    ctx = []
    for c in range(3):  # b=0 positive, b=1 uncond/negative, NAG negative
        kk = torch.randn(L, H * D, generator=g)
        vv = torch.randn(L, H * D, generator=g)
        kk = torch.from_numpy(oracle.rmsnorm_rows(kk.numpy()).reshape(L, H * D))  # cache_context's K norm
        ctx.append((kk.half(), vv.half()))
    qwb = qw.view(torch.int16).numpy().view(np.uint16)
    qn = [oracle.rmsnorm_rows(qraw[b * T:(b + 1) * T].float().numpy(), qwb).reshape(T, H * D) for b in range(B)]
    refs = [oracle.attn_f64(qn[b], ctx[b][0].float().numpy(), ctx[b][1].float().numpy(), H, npad=npad)
            for b in range(B)]
    ref_neg = oracle.attn_f64(qn[0], ctx[2][0].float().numpy(), ctx[2][1].float().numpy(), H, npad=npad)
    ref0 = oracle.nag(refs[0], ref_neg, 5.0, 2.5, 0.25)
    # fp16 semantics on the same inputs: per-attention bars, and the NAG output of emulated attentions
    emus = [oracle.attn_f16sem(qn[b], ctx[b][0].float().numpy(), ctx[b][1].float().numpy(), H, npad=npad)
            for b in range(B)]
    emu_neg = oracle.attn_f16sem(qn[0], ctx[2][0].float().numpy(), ctx[2][1].float().numpy(), H, npad=npad)
    emu0 = oracle.nag(emus[0], emu_neg, 5.0, 2.5, 0.25)
    strict = wvar is None

    kvps = [kiln_amd.kv_prepare(kk.to(DEV), vv.to(DEV), H) for kk, vv in ctx]
    out = torch.empty(B * T, H * D, dtype=torch.float16, device=DEV)
    out_neg = torch.empty(T, H * D, dtype=torch.float16, device=DEV)
    kiln_amd.cross_attn_nag(out, qraw.to(DEV), B, T, H, kvps[:2], [L, L], [npad, npad], q_norm_w=qw.to(DEV),
                            kvp_neg=kvps[2], Lk_neg=L, npad_neg=npad, out_neg=out_neg)
    torch.cuda.synchronize()
    o = out.float().cpu().numpy()
    assert_close(out_neg.float().cpu().numpy(), ref_neg, f"cross NAG-neg L={L}+{npad}",
                 **({} if strict else emulator_bar(emu_neg, ref_neg)))
    assert_close(o[T:], refs[1], f"cross b=1 L={L}+{npad}", **({} if strict else emulator_bar(emus[1], refs[1])))
    # the NAG item (item 0) at the BASELINE bar for the BASELINE inputs; the stress variant (norm weights U(1,3):
    # peaky softmax, and the blend amplifies attention error up to (2s - 1) alpha + 1 - alpha = 3x) at the
    # error that the reference's fp16 semantics themselves reach on those inputs
    bar = {} if strict else emulator_bar(emu0, ref0)
    assert_close(o[:T], ref0, f"cross+NAG b=0 fp16 out L={L}+{npad}", **bar)

    # fp32 output of the same call: the NAG item at the BASELINE bar itself (max-abs 2e-3, mean-abs 2e-4)
    out32 = torch.empty(B * T, H * D, dtype=torch.float32, device=DEV)
    neg32 = torch.empty(T, H * D, dtype=torch.float32, device=DEV)
    kiln_amd.cross_attn_nag(out32, qraw.to(DEV), B, T, H, kvps[:2], [L, L], [npad, npad], q_norm_w=qw.to(DEV),
                            kvp_neg=kvps[2], Lk_neg=L, npad_neg=npad, out_neg=neg32)
    torch.cuda.synchronize()
    o32 = out32.cpu().numpy()
    assert_close(neg32.cpu().numpy(), ref_neg, f"cross NAG-neg fp32 out L={L}+{npad}",
                 **({} if strict else emulator_bar(emu_neg, ref_neg)))
    assert_close(o32[:T], ref0, f"cross+NAG b=0 fp32 out L={L}+{npad}", **bar)


# ---- edge cases ----
@pytest.mark.parametrize("Tq,Tk,npad", [(1, 1, 0), (1, 64, 0), (65, 63, 0), (129, 65, 3), (7, 1, 100), (300, 0, 5)])
def test_edge_shapes(gpu, Tq, Tk, npad):
    q, k, v = _qkv(31, Tq, max(Tk, 1), scale_qk=1.0)
    k, v = k[:Tk], v[:Tk]
    if Tk == 0:
        ref = np.zeros((Tq, H * D), np.float32)
    else:
        ref = oracle.attn_f64(q.numpy(), k.numpy(), v.numpy(), H, npad=npad)
    out = torch.full((Tq, H * D), float("nan"), dtype=torch.float32, device=DEV)
    kd = k.to(DEV) if Tk else torch.empty(1, H * D, device=DEV)
    vd = v.to(DEV) if Tk else torch.empty(1, H * D, device=DEV)
    kiln_amd.attention(out, q.to(DEV), kd, vd, Tq, Tk, H, D, npad=npad)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), ref, f"edge Tq={Tq} Tk={Tk} npad={npad}")


@pytest.mark.parametrize("Tq,Tk,packed", [(200, 77, False), (130, 33, True), (64, 1, False), (257, 4000, True),
                                           (129, 64, True)])
def test_f16_kv_rows_past_tk_unread(gpu, Tq, Tk, packed):
    """fp16 K/V whose rows after the last key hold NaN: the prepare pass must zero-fill the ragged last half tile
    instead of reading them (a NaN there, weighted by P = 0, would still give NaN). packed: K and V are column
    slices of one [rows, 3 x 2048] buffer (row stride 6144, as a fused QKV projection writes them)."""
    q, k, v = (f16_round(t) for t in _qkv(57 + Tk, Tq, Tk, scale_qk=1.0))
    ref = oracle.attn_f64(q.numpy(), k.numpy(), v.numpy(), H)
    rows = Tk + 40
    if packed:
        buf = torch.full((rows, 3 * H * D), float("nan"), dtype=torch.float16, device=DEV)
        buf[:Tk, :H * D] = k.half().to(DEV)
        buf[:Tk, 2 * H * D:] = v.half().to(DEV)
        kd, vd = buf[:, :H * D], buf[:, 2 * H * D:]
    else:
        kd = torch.full((rows, H * D), float("nan"), dtype=torch.float16, device=DEV)
        vd = torch.full((rows, H * D), float("nan"), dtype=torch.float16, device=DEV)
        kd[:Tk] = k.half().to(DEV)
        vd[:Tk] = v.half().to(DEV)
    out = torch.empty(Tq, H * D, dtype=torch.float32, device=DEV)
    kiln_amd.attn_f16in(out, q.half().to(DEV), kd, vd, 1, Tq, Tk, H)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), ref, f"K/V past Tk Tq={Tq} Tk={Tk} packed={packed}")


@pytest.mark.parametrize("Tq,Tk,B,npad,od", [(1000, 333, 4, 5, torch.float32), (2000, 777, 2, 0, torch.float16),
                                           (1793, 64, 2, 3, torch.float32), (769, 1, 4, 0, torch.float16),
                                           (1100, 2100, 4, 7, torch.float16)])
def test_eight_wave_workgroups(gpu, Tq, Tk, B, npad, od):
    """Grids whose 256-row query tiles fill whole rounds of CUs (ceil(Tq / 256) x H x B a multiple of the CU count,
    as at config 4), or at least one round with keys >= 2048 (as config 5's self-attention), run the 8-wave kernel
    (one workgroup per CU, 8-stage ring): ragged query and key tiles, a half-empty last round, npad, both output
    types, batched items."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    t8 = ((Tq + 255) // 256) * H * B
    if t8 % cus and not (Tk >= 2048 and t8 >= cus):
        pytest.skip(f"shape does not select the 8-wave kernel on {cus} CUs")
    q, k, v = (f16_round(randn(71 + i, B * T, H * D)) for i, T in enumerate((Tq, Tk, Tk)))
    out = torch.full((B * Tq, H * D), float("nan"), dtype=od, device=DEV)
    kiln_amd.attn_f16in(out, q.half().to(DEV), k.half().to(DEV), v.half().to(DEV), B, Tq, Tk, H, npad=npad)
    torch.cuda.synchronize()
    o = out.float().cpu().numpy()
    for b in range(B):
        ref = oracle.attn_f64(q[b * Tq:(b + 1) * Tq].numpy(), k[b * Tk:(b + 1) * Tk].numpy(),
                              v[b * Tk:(b + 1) * Tk].numpy(), H, npad=npad)
        assert_close(o[b * Tq:(b + 1) * Tq], ref, f"8 waves Tq={Tq} Tk={Tk} b={b} npad={npad} out={od}")


def test_explicit_zero_keys_equal_npad(gpu):
    """npad analytic zero keys == the same zero rows present explicitly (tcflash.cuh:136-147)."""
    Tq, L, npad = 200, 40, 88
    q, k, v = _qkv(41, Tq, L, scale_qk=1.0)
    kz = torch.cat([k, torch.zeros(npad, H * D)])
    vz = torch.cat([v, torch.zeros(npad, H * D)])
    a = torch.empty(Tq, H * D, device=DEV)
    b = torch.empty(Tq, H * D, device=DEV)
    kiln_amd.attention(a, q.to(DEV), k.to(DEV), v.to(DEV), Tq, L, H, D, npad=npad)
    kiln_amd.attention(b, q.to(DEV), kz.to(DEV), vz.to(DEV), Tq, L + npad, H, D)
    torch.cuda.synchronize()
    assert_close(a.cpu().numpy(), b.cpu().numpy(), "npad vs explicit zeros", max_abs=1e-3, mean_abs=1e-4)


def test_unsupported_and_invalid(gpu):
    q = torch.zeros(8, H * 64, device=DEV)
    out = torch.zeros(8, H * 64, dtype=torch.float16, device=DEV)
    with pytest.raises(kiln_amd.KilnError) as e:
        kiln_amd.attention16(out, q, q, q, 8, 8, H, 64)
    assert e.value.status == kiln_amd.KILN_EUNSUPPORTED
    with pytest.raises(kiln_amd.KilnError) as e:
        kiln_amd.attention(torch.zeros(8, H * D, device=DEV), torch.zeros(8, H * D, device=DEV),
                           torch.zeros(8, H * D, device=DEV), torch.zeros(8, H * D, device=DEV), 8, 0, H, D)
    assert e.value.status == kiln_amd.KILN_EINVAL


# ---- exact fp32 path (causal / Dh != 128 / fp32 mode) ----
@pytest.mark.parametrize("Dh,causal,npad", [(64, False, 0), (128, True, 0), (64, True, 0), (80, False, 7)])
def test_exact_attention(gpu, Dh, causal, npad):
    Tq, Tk, Hh = 150, 150, 4
    q = randn(51, Tq, Hh * Dh)
    k = randn(52, Tk, Hh * Dh)
    v = randn(53, Tk, Hh * Dh)
    ref = oracle.attn_f64(q.numpy(), k.numpy(), v.numpy(), Hh, Dh=Dh, npad=npad, causal=causal)
    out = torch.empty(Tq, Hh * Dh, device=DEV)
    kiln_amd.attention(out, q.to(DEV), k.to(DEV), v.to(DEV), Tq, Tk, Hh, Dh, causal=causal, npad=npad)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), ref, f"exact Dh={Dh} causal={causal}", max_abs=1e-5, mean_abs=1e-6)


@pytest.mark.parametrize("Tq,Tk,Hh,causal,npad,pad", [(1000, 777, 3, False, 5, 64), (300, 300, 2, True, 0, 0),
                                                       (129, 40, 1, True, 3, 4), (33, 1, 2, False, 0, 0)])
def test_exact_attention_dh128_mfma(gpu, Tq, Tk, Hh, causal, npad, pad):
    """kiln_attn_fwd_exact at Dh = 128 (the fp32 matrix-core kernel): ragged query and key counts, causal with
    Tq != Tk, padding keys, and rows padded beyond H*128 (the head block at a column offset inside the row), against
    the float64 oracle at the exact path's bar."""
    D_ = 128
    q = randn(61, Tq, Hh * D_)
    k = randn(62, Tk, Hh * D_)
    v = randn(63, Tk, Hh * D_)
    ref = oracle.attn_f64(q.numpy(), k.numpy(), v.numpy(), Hh, Dh=D_, npad=npad, causal=causal)

    def padded(t):
        buf = torch.zeros(t.shape[0], t.shape[1] + pad, device=DEV)
        buf[:, pad // 2:pad // 2 + t.shape[1]] = t.to(DEV)
        return buf[:, pad // 2:pad // 2 + t.shape[1]]
    out_full = torch.full((Tq, Hh * D_ + pad), float("nan"), device=DEV)
    out = out_full[:, pad // 2:pad // 2 + Hh * D_]
    kiln_amd.attention_exact(out, padded(q), padded(k), padded(v), Tq, Tk, Hh, D_, causal=causal, npad=npad)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), ref, f"exact Dh=128 Tq={Tq} Tk={Tk}", max_abs=1e-5, mean_abs=1e-6)
    if pad:  # the padding columns of the output rows are untouched
        assert torch.isnan(out_full[:, :pad // 2]).all() and torch.isnan(out_full[:, pad // 2 + Hh * D_:]).all()


# ---- the bandwidth-bound ops around attention ----
def test_rmsnorm_rope_nag_kernels(gpu):
    T = 96
    x = randn(61, T, H * D)
    w = (torch.rand(D, generator=torch.Generator().manual_seed(62)) * 2 + 1).to(torch.bfloat16)
    wb = w.view(torch.int16).numpy().view(np.uint16)
    cos, sin = oracle.cosmos_rope(8, 12)
    ref = oracle.rope_half(oracle.rmsnorm_rows(x.numpy(), wb).reshape(T, H * D), H, cos, sin)
    xd = x.to(DEV)
    kiln_amd.rmsnorm(xd, xd, w.to(DEV), rows=T * H, dim=D)
    kiln_amd.rope_half(xd, T, H, D, torch.from_numpy(cos).to(DEV), torch.from_numpy(sin).to(DEV))
    torch.cuda.synchronize()
    assert_close(xd.cpu().numpy(), ref, "rmsnorm+rope", max_abs=1e-5, mean_abs=1e-6)
    c2, s2 = kiln_amd.cosmos_rope_tables(8, 12)
    assert np.array_equal(c2.numpy(), cos) and np.array_equal(s2.numpy(), sin)

    a = randn(63, T, H * D) * 0.1
    an = randn(64, T, H * D) * 0.1
    ref = oracle.nag(a.numpy(), an.numpy())
    for dt, tol in ((torch.float32, 1e-5), (torch.float16, 2e-3)):
        ad = a.to(dt).to(DEV)
        kiln_amd.nag_combine(ad, an.to(dt).to(DEV))
        torch.cuda.synchronize()
        r = oracle.nag(a.to(dt).float().numpy(), an.to(dt).float().numpy())
        assert_close(ad.float().cpu().numpy(), r, f"nag {dt}", max_abs=tol, mean_abs=tol / 10)


@pytest.mark.parametrize("dim", [2048, 520, 1000, 2056])
def test_nag_combine_widths(gpu, dim):
    """Row-per-wave vector path (dim % 8 == 0, dim <= 2048) and the general path (other widths) of the NAG
    blend (engine/src/dit.cu:295-324), fp16 and fp32, against the oracle on rows where the clamp engages
    (tau < ratio) and rows where it does not."""
    T = 37
    a = randn(65, T, dim) * 0.1
    an = randn(66, T, dim) * 0.1
    an[: T // 2] = a[: T // 2] * 0.9  # ratio < tau: no clamp
    for dt, tol in ((torch.float32, 1e-5), (torch.float16, 2e-3)):
        ad = a.to(dt).to(DEV)
        kiln_amd.nag_combine(ad, an.to(dt).to(DEV))
        torch.cuda.synchronize()
        r = oracle.nag(a.to(dt).float().numpy(), an.to(dt).float().numpy())
        assert_close(ad.float().cpu().numpy(), r, f"nag dim={dim} {dt}", max_abs=tol, mean_abs=tol / 10)


def test_prepare_multi_tile_blocks_ragged(gpu):
    """Long context (Tk = 5000: 79 tiles per head, the last holding 8 keys): the K/V prepare pass walks
    several tiles per block there, so a block's last tile is ragged and the tile-ahead loads run past Tk.
    fp32 inputs through attention16 (engine/src/gpu.h:155-156)."""
    Tq, Tk = 64, 5000
    q, k, v = _qkv(81, Tq, Tk, scale_qk=1.0)
    ref = oracle.attn_f64(q.numpy(), k.numpy(), v.numpy(), H)
    out = torch.empty(Tq, H * D, dtype=torch.float16, device=DEV)
    kiln_amd.attention16(out, q.to(DEV), k.to(DEV), v.to(DEV), Tq, Tk, H, D)
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy(), ref, f"attention16 Tq={Tq} Tk={Tk}")


def test_prepped_entry_points(gpu):
    """kiln_kv_prepare (K RMSNorm + RoPE) then kiln_attn_fwd_prepped / kiln_attn_fwd_prepped_batch (Q RMSNorm +
    RoPE in the Q load): the split form of the fused DiT call, single and batched, fp32 and fp16 outputs,
    with npad zero keys; and kiln_attn_fwd_exact called directly."""
    Hp, Wp, npad = 12, 20, 7
    T = Hp * Wp
    g = torch.Generator().manual_seed(91)
    qw = (torch.rand(D, generator=g) * 0.5 + 0.75).to(torch.bfloat16)
    kw = (torch.rand(D, generator=g) * 0.5 + 0.75).to(torch.bfloat16)
    cos, sin = oracle.cosmos_rope(Hp, Wp)
    rope = (torch.from_numpy(cos).to(DEV), torch.from_numpy(sin).to(DEV))
    qwb = qw.view(torch.int16).numpy().view(np.uint16)
    kwb = kw.view(torch.int16).numpy().view(np.uint16)
    Bn = 3
    qs = [torch.randn(T, H * D, generator=g).half() for _ in range(Bn)]
    ks = [torch.randn(T, H * D, generator=g).half() for _ in range(Bn)]
    vs = [torch.randn(T, H * D, generator=g).half() for _ in range(Bn)]
    refs = []
    for b in range(Bn):
        qn = oracle.rope_half(oracle.rmsnorm_rows(qs[b].float().numpy(), qwb).reshape(T, H * D), H, cos, sin)
        kn = oracle.rope_half(oracle.rmsnorm_rows(ks[b].float().numpy(), kwb).reshape(T, H * D), H, cos, sin)
        refs.append(oracle.attn_f64(qn, kn, vs[b].float().numpy(), H, npad=npad))
    kvps = [kiln_amd.kv_prepare(ks[b].to(DEV), vs[b].to(DEV), H, k_norm_w=kw.to(DEV), rope=rope) for b in range(Bn)]

    out = torch.empty(T, H * D, dtype=torch.float32, device=DEV)
    kiln_amd.attn_prepped(out, qs[1].to(DEV), kvps[1], T, H, npad=npad, q_norm_w=qw.to(DEV), rope=rope)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), refs[1], "attn_fwd_prepped fp32 out")

    outb = torch.empty(Bn * T, H * D, dtype=torch.float16, device=DEV)
    kiln_amd.attn_prepped_batch(outb, torch.cat(qs).to(DEV), kvps, T, T, H, npad=npad, q_norm_w=qw.to(DEV),
                                rope=rope)
    torch.cuda.synchronize()
    o = outb.float().cpu().numpy()
    for b in range(Bn):
        assert_close(o[b * T:(b + 1) * T], refs[b], f"attn_fwd_prepped_batch item {b}")

    q, k, v = _qkv(92, 50, 70, scale_qk=1.0)
    ref = oracle.attn_f64(q.numpy(), k.numpy(), v.numpy(), H, npad=3)
    oe = torch.empty(50, H * D, device=DEV)
    kiln_amd.attention_exact(oe, q.to(DEV), k.to(DEV), v.to(DEV), 50, 70, H, D, npad=3)
    torch.cuda.synchronize()
    assert_close(oe.cpu().numpy(), ref, "attn_fwd_exact Dh=128", max_abs=1e-5, mean_abs=1e-6)


# ---- modulated LayerNorm and gated residual of the DiT block ----
@pytest.mark.parametrize("rows,dim,offset", [(6912, 2048, 0), (37, 2048, 1), (64, 1000, 0), (9, 6144, 0)])
def test_layernorm_mod(gpu, rows, dim, offset):
    """kiln_layernorm_mod / _mod16 against the oracle: fp32 out to fp32 rounding (the row sums add in another
    order), fp16 out within one fp16 ulp plus that fp32 difference (values near zero have tiny ulps).
    (6912, 2048) is config 5's CFG batch (2 x 3456 tokens); offset 1 makes the rows unaligned (scalar path);
    dim 6144 exceeds the register-resident path."""
    print(f"[case] layernorm_mod rows={rows} dim={dim} offset={offset}", flush=True)
    g = torch.Generator().manual_seed(rows + dim)
    x = torch.randn(rows * dim + offset, generator=g) * 2 + 0.5
    sc = torch.randn(dim, generator=g) * 0.3
    sh = torch.randn(dim, generator=g)
    xv = x[offset:].view(rows, dim)
    ref = oracle.layernorm_mod(xv.numpy(), sc.numpy(), sh.numpy(), eps=1e-6)
    xd = x.to(DEV)[offset:].view(rows, dim)
    y32 = torch.empty(rows, dim, device=DEV)
    kiln_amd.layernorm_mod(y32, xd, sc.to(DEV), sh.to(DEV), eps=1e-6)
    y16 = torch.empty(rows, dim, dtype=torch.float16, device=DEV)
    kiln_amd.layernorm_mod(y16, xd, sc.to(DEV), sh.to(DEV), eps=1e-6)
    torch.cuda.synchronize()
    d32 = np.abs(y32.cpu().numpy() - ref)
    tol32 = 2e-5 * np.maximum(1.0, np.abs(ref))
    print(f"[parity] layernorm_mod fp32: max-abs {d32.max():.3e}", flush=True)
    assert (d32 <= tol32).all()
    r16 = ref.astype(np.float16).astype(np.float64)
    ulp = np.spacing(np.abs(r16).astype(np.float16)).astype(np.float64)
    d16 = np.abs(y16.cpu().numpy().astype(np.float64) - r16)
    print(f"[parity] layernorm_mod16: max |diff| / (ulp + fp32 bar) {float((d16 / (ulp + tol32)).max()):.2f}",
          flush=True)
    assert (d16 <= ulp * 1.0001 + tol32).all()


@pytest.mark.parametrize("rows,dim,gated", [(6912, 2048, True), (100, 2048, False), (33, 1001, True)])
def test_add_gated(gpu, rows, dim, gated):
    print(f"[case] add_gated rows={rows} dim={dim} gate={gated}", flush=True)
    g = torch.Generator().manual_seed(rows * 3 + dim)
    x = torch.randn(rows, dim, generator=g)
    y = torch.randn(rows, dim, generator=g)
    gate = torch.randn(dim, generator=g) if gated else None
    ref = oracle.add_gated(x.numpy(), y.numpy(), gate.numpy() if gated else None)
    xd = x.to(DEV)
    kiln_amd.add_gated(xd, y.to(DEV), gate.to(DEV) if gated else None)
    torch.cuda.synchronize()
    d = np.abs(xd.cpu().numpy() - ref).max()
    print(f"[parity] add_gated: max-abs {d:.3e}", flush=True)
    assert d <= 1e-6 * max(1.0, float(np.abs(ref).max()))


# ---- key-split launches (grids filling under a third of the workgroup slots) ----
@pytest.mark.parametrize("Hh,Tq,Tk,npad", [(1, 512, 4096, 100), (1, 300, 3001, 0), (2, 130, 2048, 7)])
def test_key_split_small_grid(gpu, Hh, Tq, Tk, npad):
    """Few heads and queries against many keys: the launch splits each query tile's keys into ranges (up to
    8, each >= 16 half tiles; Tk = 3001 ends on a ragged half tile) and merges the partials. Checked against
    the double-accumulation oracle, through the fp32 drop-in (library workspace) with npad."""
    print(f"[case] key split H={Hh} Tq={Tq} Tk={Tk} npad={npad}", flush=True)
    g = torch.Generator().manual_seed(Tq + Tk)
    q = torch.randn(Tq, Hh * D, generator=g)
    k = torch.randn(Tk, Hh * D, generator=g)
    v = torch.randn(Tk, Hh * D, generator=g)
    ref = oracle.attn_f64(q.numpy(), k.numpy(), v.numpy(), Hh, npad=npad)
    out = torch.full((Tq, Hh * D), float("nan"), dtype=torch.float32, device=DEV)
    kiln_amd.attention(out, q.to(DEV), k.to(DEV), v.to(DEV), Tq, Tk, Hh, D, npad=npad)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), ref, f"key split H={Hh} Tq={Tq} Tk={Tk} npad={npad}")


def test_key_split_tp_share_config4(gpu):
    """One GPU's share of config 4 under 8-way head parallelism (H=2 of 16, T=4096, B=2, QK-norm + RoPE,
    fp16): 128 query-tile units, split 4 ways. Sampled query rows of both items against the oracle; the
    caller's workspace sized by kiln_dit_self_attn_workspace_bytes (split) and one only large enough for
    the prepared K/V (unsplit) give outputs within fp16 rounding of each other."""
    Hh, B, Hp, Wp = 2, 2, 64, 64
    T = Hp * Wp
    print(f"[case] TP share H={Hh} T={T} B={B}", flush=True)
    g = torch.Generator().manual_seed(77)
    q, k, v = (torch.randn(B * T, Hh * D, generator=g).half() for _ in range(3))
    qw = (torch.rand(D, generator=g) * 0.5 + 0.75).to(torch.bfloat16)
    kw = (torch.rand(D, generator=g) * 0.5 + 0.75).to(torch.bfloat16)
    c, s = oracle.cosmos_rope(Hp, Wp)
    rope = (torch.from_numpy(c).to(DEV), torch.from_numpy(s).to(DEV))
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    full = kiln_amd.dit_self_attn_workspace_bytes(B, T, Hh)
    small = B * kiln_amd.kv_prepped_bytes(T, Hh)
    assert full > small, "expected the split workspace on this device"
    outs = []
    for nbytes in (full, small):
        ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        out = torch.empty(B * T, Hh * D, dtype=torch.float16, device=DEV)
        kiln_amd.dit_self_attn(out, qd, kd, vd, B, T, Hh, qw.to(DEV), kw.to(DEV), rope, workspace=ws)
        torch.cuda.synchronize()
        outs.append(out.float().cpu().numpy())
    qwb = qw.view(torch.int16).numpy().view(np.uint16)
    kwb = kw.view(torch.int16).numpy().view(np.uint16)
    rows = np.arange(0, T, 29)
    for b in range(B):
        sl = slice(b * T, (b + 1) * T)
        qn = oracle.rope_half(oracle.rmsnorm_rows(q[sl].float().numpy(), qwb).reshape(T, Hh * D), Hh, c, s)
        kn = oracle.rope_half(oracle.rmsnorm_rows(k[sl].float().numpy(), kwb).reshape(T, Hh * D), Hh, c, s)
        ref = oracle.attn_f64(np.ascontiguousarray(qn[rows]), kn, v[sl].float().numpy(), Hh)
        assert_close(outs[0][sl][rows], ref, f"TP share split, item {b}")
        assert_close(outs[1][sl][rows], ref, f"TP share unsplit, item {b}")
    assert np.abs(outs[0] - outs[1]).max() <= 2e-3
