"""Pins the CPU oracle (oracle/oracle.c) with checks that do not restate its own formulas:
library routines (torch float64 attention, torch rms_norm, complex rotation), committed fixtures
(torch.randn), closed forms and invariants, and brute-force special cases. CPU only.
"""
import json
import os

import numpy as np
import pytest
import torch

import oracle

HERE = os.path.dirname(os.path.abspath(__file__))
rng = np.random.default_rng(1234)


def sdpa64(q, k, v, H, Dh, causal=False):
    """torch float64 softmax attention per head (the library routine)."""
    Tq, Tk = q.shape[0], k.shape[0]
    qt = torch.from_numpy(q.astype(np.float64)).view(Tq, H, Dh).transpose(0, 1)
    kt = torch.from_numpy(k.astype(np.float64)).view(Tk, H, Dh).transpose(0, 1)
    vt = torch.from_numpy(v.astype(np.float64)).view(Tk, H, Dh).transpose(0, 1)
    o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, is_causal=causal)
    return o.transpose(0, 1).reshape(Tq, H * Dh).numpy()


# ---------------------------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("Tq,Tk,H,Dh", [(7, 5, 2, 128), (33, 70, 3, 128), (16, 16, 4, 64), (5, 1, 2, 80)])
def test_attn_f64_matches_torch_float64(Tq, Tk, H, Dh):
    q, k, v = (rng.standard_normal((n, H * Dh)).astype(np.float32) for n in (Tq, Tk, Tk))
    np.testing.assert_allclose(oracle.attn_f64(q, k, v, H, Dh), sdpa64(q, k, v, H, Dh), atol=1e-6, rtol=1e-6)


def test_attn_f64_causal_matches_torch():
    T, H, Dh = 24, 2, 64
    q, k, v = (rng.standard_normal((T, H * Dh)).astype(np.float32) for _ in range(3))
    np.testing.assert_allclose(oracle.attn_f64(q, k, v, H, Dh, causal=True), sdpa64(q, k, v, H, Dh, causal=True),
                               atol=1e-6, rtol=1e-6)


@pytest.mark.parametrize("npad", [1, 26, 486])
def test_npad_equals_explicit_zero_keys(npad):
    """npad analytic zero keys (flash_test.cu:15,22; kernels.cu:815-817) == zero K/V rows present."""
    Tq, Tk, H, Dh = 9, 26, 2, 128
    q = rng.standard_normal((Tq, H * Dh)).astype(np.float32) * 1.5
    k = rng.standard_normal((Tk, H * Dh)).astype(np.float32) * 1.5
    v = rng.standard_normal((Tk, H * Dh)).astype(np.float32)
    kz = np.concatenate([k, np.zeros((npad, H * Dh), np.float32)])
    vz = np.concatenate([v, np.zeros((npad, H * Dh), np.float32)])
    full = sdpa64(q, kz, vz, H, Dh)
    np.testing.assert_allclose(oracle.attn_f64(q, k, v, H, Dh, npad=npad), full, atol=1e-6, rtol=1e-6)
    np.testing.assert_allclose(oracle.ref_attn_f32(q, k, v, H, Dh, npad=npad), full, atol=2e-5, rtol=1e-4)


def test_ref_attn_f32_matches_torch():
    Tq, Tk, H = 40, 97, 2
    q, k, v = (rng.standard_normal((n, H * 128)).astype(np.float32) for n in (Tq, Tk, Tk))
    np.testing.assert_allclose(oracle.ref_attn_f32(q, k, v, H), sdpa64(q, k, v, H, 128), atol=2e-5, rtol=1e-4)


def test_attention_invariants():
    H, Dh = 2, 128
    q = rng.standard_normal((6, H * Dh)).astype(np.float32)
    k = rng.standard_normal((11, H * Dh)).astype(np.float32)
    v = rng.standard_normal((11, H * Dh)).astype(np.float32)
    # one key: the output is that key's value row
    np.testing.assert_allclose(oracle.attn_f64(q, k[:1], v[:1], H), np.repeat(v[:1], 6, 0), atol=1e-7)
    # identical keys: uniform weights, the output is the mean of V
    kk = np.repeat(k[:1], 11, 0)
    np.testing.assert_allclose(oracle.attn_f64(q, kk, v, H), np.repeat(v.mean(0, keepdims=True), 6, 0), atol=1e-6)
    # permuting keys together with values leaves the output unchanged
    p = rng.permutation(11)
    np.testing.assert_allclose(oracle.attn_f64(q, k[p], v[p], H), oracle.attn_f64(q, k, v, H), atol=1e-6)
    # V = ones -> 1 without padding, Tk/(Tk + npad e^{-m}) with padding (m = max(0, max score))
    ones = np.ones_like(v)
    np.testing.assert_allclose(oracle.attn_f64(q, k, ones, H), 1.0, atol=1e-6)


def test_f16sem_emulator_special_cases():
    """The fp16-semantics emulator (tcflash.cuh:33-156): exact special cases and the fp16 error budget."""
    H = 2
    q = rng.standard_normal((8, H * 128)).astype(np.float32)
    v = rng.standard_normal((5, H * 128)).astype(np.float32)
    k = rng.standard_normal((5, H * 128)).astype(np.float32)
    v16 = v.astype(np.float16).astype(np.float32)
    # one key: p = 2^0 = 1 exactly, output = fp16(V0) exactly (fp32 out) and after fp16 rounding
    np.testing.assert_array_equal(oracle.attn_f16sem(q, k[:1], v[:1], H, out16=False), np.repeat(v16[:1], 8, 0))
    # identical keys: all p = 1, output = fp32 mean of fp16(V) (sum order aside)
    kk = np.repeat(k[:1], 5, 0)
    np.testing.assert_allclose(oracle.attn_f16sem(q, kk, v, H, out16=False),
                               np.repeat(v16.mean(0, keepdims=True), 8, 0), atol=2e-7)
    # error against exact attention stays inside the fp16 budget of Q/K/P rounding
    q, k, v = (rng.standard_normal((n, H * 128)).astype(np.float32) for n in (64, 300, 300))
    d = np.abs(oracle.attn_f16sem(q, k, v, H, out16=False) - oracle.attn_f64(q, k, v, H))
    assert d.max() < 2e-3 and d.mean() < 1e-4
    # fp16 output rounding: out16 = fp16(out32)
    o32 = oracle.attn_f16sem(q, k, v, H, out16=False)
    np.testing.assert_array_equal(oracle.attn_f16sem(q, k, v, H, out16=True), o32.astype(np.float16).astype(np.float32))


def test_f16sem_npad_single_key():
    """Tk = 1, npad zero keys: scores relative to m' = max(m, 0) (tcflash.cuh:142-146), closed form."""
    H = 1
    q = rng.standard_normal((3, 128)).astype(np.float32)
    k = rng.standard_normal((1, 128)).astype(np.float32)
    v = rng.standard_normal((1, 128)).astype(np.float32)
    npad = 7
    q16 = (q * np.float32(1.4426950408889634 / np.sqrt(128))).astype(np.float16).astype(np.float64)
    s = q16 @ k.astype(np.float16).astype(np.float64).T  # base-2 score of the one key
    w = 1.0 / (1.0 + npad * np.exp2(-s))                # its softmax weight next to npad zero keys
    expect = w * v.astype(np.float16).astype(np.float64)
    np.testing.assert_allclose(oracle.attn_f16sem(q, k, v, H, npad=npad, out16=False), expect, rtol=2e-6, atol=1e-7)


# ---------------------------------------------------------------------------------------------
# QK-RMSNorm, RoPE, Cosmos RoPE tables
# ---------------------------------------------------------------------------------------------
def test_rmsnorm_matches_torch_and_unit_rms():
    x = rng.standard_normal((50, 128)).astype(np.float32) * 3
    w = (rng.random(128) * 2 + 1).astype(np.float32)
    wb = torch.from_numpy(w).to(torch.bfloat16)
    wbits = wb.view(torch.int16).numpy().view(np.uint16)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x), (128,), wb.float(), eps=1e-6).numpy()
    np.testing.assert_allclose(oracle.rmsnorm_rows(x, wbits), ref, rtol=2e-6, atol=1e-6)
    y = oracle.rmsnorm_rows(x)  # w = 1: every row has RMS 1 (up to eps)
    np.testing.assert_allclose(np.sqrt((y.astype(np.float64) ** 2).mean(1)), 1.0, atol=1e-6)


def test_rope_half_is_complex_rotation():
    T, H = 9, 3
    x = rng.standard_normal((T, H * 128)).astype(np.float32)
    ang = rng.random((T, 64)) * 20
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    y = oracle.rope_half(x, H, c, s)
    z = (x.reshape(T, H, 2, 64)[:, :, 0] + 1j * x.reshape(T, H, 2, 64)[:, :, 1]) * (c + 1j * s)[:, None, :]
    np.testing.assert_allclose(y.reshape(T, H, 2, 64)[:, :, 0], z.real, atol=2e-6)
    np.testing.assert_allclose(y.reshape(T, H, 2, 64)[:, :, 1], z.imag, atol=2e-6)
    # rotation keeps each pair's norm
    np.testing.assert_allclose(np.abs(z), np.hypot(y.reshape(T, H, 2, 64)[:, :, 0], y.reshape(T, H, 2, 64)[:, :, 1]),
                               rtol=1e-5)


def cosmos_rope_f64(Hp, Wp, head_dim=128, extrapolation=4.0):
    """Independent float64 statement of the published Cosmos-Predict2 3D RoPE for one frame: per head,
    dim_h = dim_w = head_dim//6*2 frequencies for height and width, the rest temporal; NTK-scaled
    theta = 10000 * ratio^(dim/(dim-2)); the rotated half-vector is [t | h | w]."""
    dim_h = head_dim // 6 * 2
    dim_t = head_dim - 2 * dim_h
    theta = 10000.0 * extrapolation ** (dim_h / (dim_h - 2))
    fh = theta ** (-np.arange(0, dim_h, 2) / dim_h)
    ys, xs = np.meshgrid(np.arange(Hp), np.arange(Wp), indexing="ij")
    ang = np.zeros((Hp * Wp, head_dim // 2))
    ang[:, dim_t // 2: dim_t // 2 + dim_h // 2] = ys.reshape(-1, 1) * fh
    ang[:, dim_t // 2 + dim_h // 2:] = xs.reshape(-1, 1) * fh
    return np.cos(ang), np.sin(ang)


@pytest.mark.parametrize("Hp,Wp", [(32, 48), (64, 64), (48, 72)])
def test_cosmos_rope_tables(Hp, Wp):
    c, s = oracle.cosmos_rope(Hp, Wp)
    rc, rs = cosmos_rope_f64(Hp, Wp)
    np.testing.assert_allclose(c, rc, atol=3e-5)
    np.testing.assert_allclose(s, rs, atol=3e-5)
    assert np.all(c[0] == 1) and np.all(s[0] == 0)           # position 0 is the identity
    assert np.all(c[:, :22] == 1) and np.all(s[:, :22] == 0)  # temporal frequencies: identity for one frame


# ---------------------------------------------------------------------------------------------
# NAG
# ---------------------------------------------------------------------------------------------
def test_nag_hand_computed_row():
    """s=5, tau=2.5, alpha=0.25 on a 4-element row, by hand:
    z+ = [1, -2, 0.5, 0], z- = [0.5, 1, -1, 2]
    g = 5 z+ - 4 z- = [3, -14, 6.5, -8]; |g|_1 = 31.5; |z+|_1 = 3.5; ratio = 9 > 2.5 -> k = 2.5/9
    out = 0.25 k g + 0.75 z+"""
    zp = np.array([[1, -2, 0.5, 0]], np.float32)
    zn = np.array([[0.5, 1, -1, 2]], np.float32)
    k = 2.5 / 9.0
    g = np.array([3, -14, 6.5, -8])
    expect = 0.25 * k * g + 0.75 * zp[0]
    np.testing.assert_allclose(oracle.nag(zp, zn), expect[None], rtol=1e-6)


def test_nag_invariants():
    zp = rng.standard_normal((5, 64)).astype(np.float32)
    zn = rng.standard_normal((5, 64)).astype(np.float32)
    np.testing.assert_allclose(oracle.nag(zp, zn, s=1.0), zp, atol=1e-6)       # g = z+ -> identity
    np.testing.assert_allclose(oracle.nag(zp, zn, alpha=0.0), zp, atol=0)      # no blend
    # no clamp when the ratio stays below tau: plain extrapolation blend
    out = oracle.nag(zp, zn, s=1.2, tau=100.0, alpha=0.5)
    np.testing.assert_allclose(out, 0.5 * (1.2 * zp - 0.2 * zn) + 0.5 * zp, atol=1e-6)


# ---------------------------------------------------------------------------------------------
# torch_randn and fp16 conversion
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("seed", [0, 42, 123456789])
def test_torch_randn_matches_torch_fixture(seed):
    """torch_randn (pipeline.cu:17-64) against torch.randn bits committed in tests/golden: the MT19937
    stream and the 16-value Box-Muller layout must agree exactly; only libm's log/cos/sin may differ by a
    few ulp from torch's vectorized ones."""
    with open(os.path.join(HERE, "golden", f"randn_seed{seed}.json")) as f:
        d = json.load(f)
    ref = np.array([int(b, 16) for b in d["bits"]], dtype=np.uint32).view(np.float32)
    got = oracle.torch_randn(seed, d["n"])
    ulp = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert ulp.max() <= 4, f"max {ulp.max()} ulp"
    assert (ulp == 0).mean() > 0.7


def test_f16_rounding_matches_numpy():
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10,
                        np.array([0, -0.0, 65504, 65519.99, 65520, -70000, 6e-8, 2.98e-8, 2.99e-8, 5.96e-8,
                                  1e-5, np.inf, -np.inf, 0.1, 1 / 3], np.float32),
                        (rng.standard_normal(2000) * 1e-6).astype(np.float32)])
    np.testing.assert_array_equal(oracle.to_f16_bits(x), x.astype(np.float16).view(np.uint16))


# ---- modulated LayerNorm and gated residual of the DiT block ----
def test_layernorm_mod_matches_torch_float64():
    """oracle.layernorm_mod against an independent float64 statement: torch layer_norm without affine,
    then * (1 + scale) + shift (engine/src/kernels.cu:678-697)."""
    rng = np.random.default_rng(7)
    for rows, dim in [(3, 2048), (5, 1000), (2, 7)]:
        x = (rng.standard_normal((rows, dim)) * 3 + 1.5).astype(np.float32)
        sc = (rng.standard_normal(dim) * 0.2).astype(np.float32)
        sh = rng.standard_normal(dim).astype(np.float32)
        got = oracle.layernorm_mod(x, sc, sh, eps=1e-6)
        ref = (torch.nn.functional.layer_norm(torch.from_numpy(x).double(), (dim,), eps=1e-6)
               * (1 + torch.from_numpy(sc).double()) + torch.from_numpy(sh).double()).numpy()
        assert np.abs(got - ref).max() <= 2e-5 * max(1.0, np.abs(ref).max())


def test_layernorm_mod_unmodulated_is_standardized():
    rng = np.random.default_rng(8)
    x = (rng.standard_normal((4, 512)) * 5 - 2).astype(np.float32)
    y = oracle.layernorm_mod(x, np.zeros(512, np.float32), np.zeros(512, np.float32), eps=0.0).astype(np.float64)
    assert np.abs(y.mean(axis=1)).max() < 1e-5
    assert np.abs(y.var(axis=1) - 1).max() < 1e-4


def test_add_gated_cases():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((3, 64)).astype(np.float32)
    y = rng.standard_normal((3, 64)).astype(np.float32)
    np.testing.assert_array_equal(oracle.add_gated(x, y), x + y)
    np.testing.assert_array_equal(oracle.add_gated(x, y, np.zeros(64, np.float32)), x)
    g = np.arange(64, dtype=np.float32) / 8
    np.testing.assert_allclose(oracle.add_gated(x, y, g), x + g[None, :] * y, rtol=0, atol=1e-6)


def _f16(rng, shape, scale=1.0):
    """Random fp16 bit patterns and their exact float64 values."""
    v = (rng.standard_normal(shape) * scale).astype(np.float16)
    return v.view(np.uint16), v.astype(np.float64)


def test_linear16_matches_numpy_float64():
    """oracle.linear16's product against numpy float64 matmul on the same fp16 values, every epilogue
    (engine/src/kernels.cu:573-609, tcgemm16.cuh:145-175)."""
    import math
    rng = np.random.default_rng(21)
    T, rows, cols = 37, 256, 96
    xb, x = _f16(rng, (T, cols))
    wb, w = _f16(rng, (rows, cols), cols ** -0.5)
    acc = x @ w.T
    y0 = rng.standard_normal((T, rows)).astype(np.float32)
    got = oracle.linear16(xb, wb, oracle.EPI_F32)
    np.testing.assert_allclose(got, acc, rtol=1e-6, atol=1e-6)
    got = oracle.linear16(xb, wb, oracle.EPI_F32, y=y0, beta=0.5)
    np.testing.assert_allclose(got, acc + 0.5 * y0, rtol=1e-6, atol=1e-6)
    got = oracle.linear16(xb, wb, oracle.EPI_F16).view(np.float16).astype(np.float64)
    np.testing.assert_array_equal(got, acc.astype(np.float32).astype(np.float16).astype(np.float64))
    gelu = np.vectorize(lambda v: 0.5 * v * (1 + math.erf(v / math.sqrt(2))))(acc)
    got = oracle.linear16(xb, wb, oracle.EPI_GELU16).view(np.float16).astype(np.float64)
    np.testing.assert_array_equal(got, gelu.astype(np.float32).astype(np.float16).astype(np.float64))
    g = rng.standard_normal(rows).astype(np.float32)
    got = oracle.linear16(xb, wb, oracle.EPI_RESID, y=y0, gate=g)
    np.testing.assert_allclose(got, y0 + g[None, :] * acc, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(oracle.linear16(xb, wb, oracle.EPI_RESID, y=y0), y0 + acc, rtol=1e-6, atol=1e-6)
    np.testing.assert_array_equal(oracle.linear16(xb, wb, oracle.EPI_RESID, y=y0, gate=np.zeros(rows, np.float32)), y0)


def test_linear16_lora_is_concatenated_product():
    """The folded second product equals one product over [x | a2] and [w | w2] (kernels.cu:564-566)."""
    rng = np.random.default_rng(22)
    T, rows, cols, k2 = 19, 128, 64, 32
    xb, _ = _f16(rng, (T, cols))
    wb, _ = _f16(rng, (rows, cols), 0.2)
    ab, _ = _f16(rng, (T, k2))
    vb, _ = _f16(rng, (rows, k2), 0.2)
    got = oracle.linear16(xb, wb, oracle.EPI_F32, a2=ab, w2=vb)
    ref = oracle.linear16(np.concatenate([xb, ab], 1), np.concatenate([wb, vb], 1), oracle.EPI_F32)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-6)


def test_linear16_gelu_special_values():
    """GELU(0) = 0, GELU(v) = v for large v, GELU(-v) = 0 for large v, GELU(1) = Phi(1) from its tabulated
    value 0.8413447460685429."""
    # one-column products: x = v, w = 1
    vals = np.array([0.0, 1.0, 12.0, -12.0, 4.0], np.float16)
    xb = vals.reshape(-1, 1).repeat(32, 1)
    xb[:, 1:] = 0
    wb = np.zeros((128, 32), np.float16)
    wb[:, 0] = 1
    got = oracle.linear16(xb.view(np.uint16), wb.view(np.uint16), oracle.EPI_GELU16).view(np.float16)[:, 0]
    ref = np.array([0.0, 0.8413447460685429, 12.0, 0.0, 4.0 * 0.9999683287581669], np.float64)
    np.testing.assert_array_equal(got, ref.astype(np.float16))


def _bf16_bits(a):
    """float32 -> bf16 bit patterns by truncation (exactly representable test weights)."""
    return (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def _bf16_vals(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def test_matvec_and_linear_f32_match_numpy():
    rng = np.random.default_rng(41)
    W = _bf16_bits(rng.standard_normal((37, 200)))
    x = rng.standard_normal(200).astype(np.float32)
    add = rng.standard_normal(37).astype(np.float32)
    np.testing.assert_allclose(oracle.matvec_bf16(W, x, add), _bf16_vals(W) @ x + add, rtol=1e-6, atol=1e-6)
    X = rng.standard_normal((9, 200)).astype(np.float32)
    np.testing.assert_allclose(oracle.linear_f32(X, W), X.astype(np.float64) @ _bf16_vals(W).T, rtol=1e-6, atol=1e-6)


def test_patchify_positions_and_round_trip():
    """Hand-computed positions (engine/src/dit.cu:174-191) and unpatchify o (patchify with its features reordered
    from 4c + 2m + n to 32m + 16n + c) = identity."""
    Hl, Wl = 6, 8
    lat = np.random.default_rng(42).standard_normal((16, Hl, Wl)).astype(np.float32)
    tok = oracle.patchify(lat)
    assert tok.shape == (12, 68) and (tok[:, 64:] == 0).all()
    # token t = 5 is patch row 1, column 1 (Wp = 4): pixel (2 + m, 2 + n); feature 4c + 2m + n
    assert tok[5, 4 * 3 + 2 * 1 + 0] == lat[3, 3, 2]
    assert tok[5, 4 * 15 + 1] == lat[15, 2, 3]
    c, m, n = np.meshgrid(np.arange(16), np.arange(2), np.arange(2), indexing="ij")
    reorder = np.zeros(64, np.int64)
    reorder[(32 * m + 16 * n + c).ravel()] = (4 * c + 2 * m + n).ravel()
    np.testing.assert_array_equal(oracle.unpatchify(tok[:, reorder], Hl, Wl), lat)
