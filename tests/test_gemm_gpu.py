"""GPU parity of kiln_linear16 (the DiT's fp16 linear layers with fused epilogues) through the C ABI.

Reference: linear16 / tc16::k_gemm16 (engine/src/kernels.cu:573-609, engine/src/tcgemm16.cuh:1-200). Checked
against oracle.linear16 (double accumulation over the same fp16 values) on seeded inputs, and at the DiT's
full sizes against a plain PyTorch fp32 matmul of the same fp16 values.

Bar: the GPU accumulates in fp32 in its own order, so an fp32 output may differ from the exact sum by the
rounding of an fp32 accumulation: |err| <= sqrt(K) * 2^-21 * sum_k |x_k w_k| + 1e-7 (about 20x the expected
random-walk error at K = 2048). fp16 outputs may in addition round to the neighbouring fp16 value: + 1 fp16
ulp of the reference. RESID adds the fp32 rounding of the residual sum: + 1 fp32 ulp of the result.
"""
import numpy as np
import pytest
import torch

import kiln_amd
import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
EPIS = [oracle.EPI_F32, oracle.EPI_F16, oracle.EPI_GELU16, oracle.EPI_RESID]


def _f16(gen, shape, scale=1.0):
    return (torch.randn(shape, generator=gen, dtype=torch.float32) * scale).to(torch.float16)


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _abs_acc(x, w, a2=None, w2=None):
    r = x.double().abs() @ w.double().abs().T
    if a2 is not None:
        r += a2.double().abs() @ w2.double().abs().T
    return r.numpy()


def _ulp16(r):
    return 2.0 ** (np.floor(np.log2(np.maximum(np.abs(r), 2.0 ** -14))) - 10)


def _check(epi, got, ref, absacc, K, gate=None):
    """got / ref as float64 arrays of the same shape; see the module docstring for the bar."""
    bar = np.sqrt(K) * 2.0 ** -21 * absacc + 1e-7
    if epi == oracle.EPI_RESID:
        g = np.abs(gate)[None, :] if gate is not None else 1.0
        bar = bar * g + np.abs(ref) * 2.0 ** -23
    elif epi in (oracle.EPI_F16, oracle.EPI_GELU16):
        bar = bar + _ulp16(ref)
    err = np.abs(got - ref)
    assert np.isfinite(got).all()
    worst = np.unravel_index(np.argmax(err - bar), err.shape)
    assert (err <= bar).all(), f"epi {epi}: err {err[worst]:.3e} > bar {bar[worst]:.3e} at {worst}"


def _run(epi, T, rows, cols, k2=0, ldy=None, y_off=0, beta=0.0, with_gate=True, seed=0):
    gen = torch.Generator().manual_seed(seed)
    x = _f16(gen, (T, cols))
    w = _f16(gen, (rows, cols), cols ** -0.5)
    a2 = _f16(gen, (T, k2)) if k2 else None
    w2 = _f16(gen, (rows, k2), 0.1) if k2 else None
    ldy = ldy or rows
    fp32_out = epi in (oracle.EPI_F32, oracle.EPI_RESID)
    dt = torch.float32 if fp32_out else torch.float16
    y0 = torch.randn((T, rows), generator=gen) if fp32_out else torch.zeros((T, rows))
    gate = torch.randn(rows, generator=gen) if (epi == oracle.EPI_RESID and with_gate) else None
    # output rows of ldy elements starting y_off elements into the buffer
    buf = torch.full((T * ldy + y_off + 8,), float("nan"), dtype=dt, device=DEV)
    y = buf[y_off:y_off + T * ldy].view(T, ldy)[:, :rows]
    y.copy_(y0.to(dt))
    args = dict(epi=epi, gate=gate.to(DEV) if gate is not None else None, beta=beta)
    if k2:
        args.update(a2=a2.to(DEV), w2=w2.to(DEV))
    kiln_amd.linear16(y, x.to(DEV), w.to(DEV), **args)
    torch.cuda.synchronize()
    got = y.float().cpu().double().numpy()
    ref = oracle.linear16(_bits(x), _bits(w), epi, y=y0.numpy() if fp32_out else None,
                          gate=gate.numpy() if gate is not None else None, beta=beta,
                          a2=_bits(a2) if k2 else None, w2=_bits(w2) if k2 else None)
    if not fp32_out:
        ref = ref.view(np.float16)
    _check(epi, got, ref.astype(np.float64), _abs_acc(x, w, a2, w2), cols + k2,
           gate.numpy() if gate is not None else None)
    if ldy > rows:  # the padding columns of every row are untouched
        pad = buf[y_off:y_off + T * ldy].view(T, ldy)[:, rows:]
        assert torch.isnan(pad.float()).all()
    return got


@pytest.mark.parametrize("epi", EPIS)
def test_linear16_small_ragged(gpu, epi):
    """T = 37 (one partial row tile), K = 96 (three k tiles: fewer than the ring's four stages)."""
    _run(epi, 37, 256, 96)


@pytest.mark.parametrize("epi", EPIS)
def test_linear16_tails(gpu, epi):
    """T = 300 (two row tiles, the second ragged), rows = 384 (a half-empty column tile), K = 1024."""
    _run(epi, 300, 384, 1024, seed=1)


@pytest.mark.parametrize("epi", [oracle.EPI_F32, oracle.EPI_RESID])
def test_linear16_lora_second_product(gpu, epi):
    """The folded LoRA product (k2 = 64) after K = 512 (kernels.cu:564-566)."""
    _run(epi, 129, 256, 512, k2=64, seed=2)


def test_linear16_beta_and_null_gate(gpu):
    _run(oracle.EPI_F32, 64, 128, 64, beta=0.5, seed=3)
    _run(oracle.EPI_RESID, 64, 128, 64, with_gate=False, seed=4)


@pytest.mark.parametrize("epi", EPIS)
def test_linear16_strided_unaligned_output(gpu, epi):
    """ldy = rows + 6 and the output base 2 elements into its buffer: the element-pair store path; the
    padding columns stay untouched."""
    _run(epi, 70, 256, 128, ldy=262, y_off=2, seed=5)


def test_linear16_single_k_tile(gpu):
    _run(oracle.EPI_F32, 5, 128, 32, seed=6)


def test_linear16_rejects_ineligible(gpu):
    x = torch.zeros((4, 40), dtype=torch.float16, device=DEV)
    w = torch.zeros((128, 40), dtype=torch.float16, device=DEV)
    y = torch.zeros((4, 128), device=DEV)
    with pytest.raises(kiln_amd.KilnError, match="status 2"):
        kiln_amd.linear16(y, x, w)  # cols % 32 != 0
    w = torch.zeros((96, 64), dtype=torch.float16, device=DEV)
    with pytest.raises(kiln_amd.KilnError, match="status 2"):
        kiln_amd.linear16(y, torch.zeros((4, 64), dtype=torch.float16, device=DEV), w)  # rows % 128 != 0


# DiT 2B shapes at config 5's batch (T = 2 x 3456): QKV / O (2048 x 2048), MLP up (8192 x 2048, GELU),
# MLP down (2048 x 8192, gated residual).
DIT = [(oracle.EPI_F32, 2048, 2048), (oracle.EPI_GELU16, 8192, 2048), (oracle.EPI_RESID, 2048, 8192)]


@pytest.mark.parametrize("epi,rows,cols", DIT)
def test_linear16_dit_shapes(gpu, epi, rows, cols):
    """Full size against torch fp32 on all outputs; 96 sampled rows against the double oracle."""
    T = 6912
    gen = torch.Generator().manual_seed(7)
    x = _f16(gen, (T, cols)).to(DEV)
    w = _f16(gen, (rows, cols), cols ** -0.5).to(DEV)
    fp32_out = epi != oracle.EPI_GELU16
    y0 = torch.randn((T, rows), generator=gen).to(DEV)
    gate = torch.randn(rows, generator=gen).to(DEV) if epi == oracle.EPI_RESID else None
    y = y0.clone() if fp32_out else torch.empty((T, rows), dtype=torch.float16, device=DEV)
    kiln_amd.linear16(y, x, w, epi=epi, gate=gate)
    acc = x.float() @ w.float().T
    absacc = x.float().abs() @ w.float().abs().T
    if epi == oracle.EPI_RESID:
        ref = y0 + gate[None, :] * acc
        bar = (np.sqrt(cols) * 2.0 ** -21 * absacc + 1e-7) * gate.abs()[None, :] + ref.abs() * 2.0 ** -23
    elif epi == oracle.EPI_GELU16:
        ref = (0.5 * acc * (1 + torch.erf(acc * 0.7071067811865476))).half().float()
        bar = np.sqrt(cols) * 2.0 ** -21 * absacc + 1e-7
        bar = bar + torch.from_numpy(_ulp16(ref.cpu().numpy())).to(DEV)
    else:
        ref = acc
        bar = np.sqrt(cols) * 2.0 ** -21 * absacc + 1e-7
    # torch's fp32 matmul is itself an fp32 accumulation: allow its rounding too (twice the bar)
    err = (y.float() - ref).abs()
    assert torch.isfinite(y.float()).all()
    assert (err <= 2 * bar).all(), f"max err/bar {(err / bar).max().item():.3f}"
    idx = torch.randperm(T, generator=gen)[:96]
    xs = x[idx.to(DEV)].cpu()
    ref_o = oracle.linear16(_bits(xs), _bits(w.cpu()), epi, y=y0[idx.to(DEV)].cpu().numpy() if fp32_out else None,
                            gate=gate.cpu().numpy() if gate is not None else None)
    if not fp32_out:
        ref_o = ref_o.view(np.float16)
    _check(epi, y[idx.to(DEV)].float().cpu().double().numpy(), ref_o.astype(np.float64),
           _abs_acc(xs, w.cpu()), cols, gate.cpu().numpy() if gate is not None else None)


@pytest.mark.parametrize("epi", [oracle.EPI_F32, oracle.EPI_GELU16])
def test_linear16_tall_grid(gpu, epi):
    """T = 8192, rows = 2048: 256-row tiles fill the 256 CUs exactly (the 224-row tiles of T = 6912 would
    need a second round), so this grid takes the other tile height. 128 sampled rows against the oracle."""
    T, rows, cols = 8192, 2048, 256
    gen = torch.Generator().manual_seed(8)
    x = _f16(gen, (T, cols))
    w = _f16(gen, (rows, cols), cols ** -0.5)
    dt = torch.float16 if epi == oracle.EPI_GELU16 else torch.float32
    y = torch.zeros((T, rows), dtype=dt, device=DEV)
    kiln_amd.linear16(y, x.to(DEV), w.to(DEV), epi=epi)
    idx = torch.randperm(T, generator=gen)[:128]
    ref = oracle.linear16(_bits(x[idx]), _bits(w), epi)
    if epi == oracle.EPI_GELU16:
        ref = ref.view(np.float16)
    _check(epi, y[idx.to(DEV)].float().cpu().double().numpy(), ref.astype(np.float64), _abs_acc(x[idx], w), cols)


@pytest.mark.parametrize("T,rows,cols,k2", [(37, 256, 96, 0), (300, 384, 1024, 0), (129, 256, 512, 64), (8192, 2048, 256, 0)])
def test_linear16_prepped_weight_bit_identical(gpu, T, rows, cols, k2):
    """kiln_linear16_prepped on the prepared weight gives bit-identical outputs to kiln_linear16 on the fp16
    weight, every epilogue (the same products in the same order; only the weight's memory layout differs)."""
    gen = torch.Generator().manual_seed(9)
    x = _f16(gen, (T, cols)).to(DEV)
    w = _f16(gen, (rows, cols), cols ** -0.5).to(DEV)
    a2 = _f16(gen, (T, k2)).to(DEV) if k2 else None
    w2 = _f16(gen, (rows, k2), 0.1).to(DEV) if k2 else None
    wp = kiln_amd.linear16_prepare_weight(w)
    gate = torch.randn(rows, generator=gen).to(DEV)
    for epi in EPIS:
        dt = torch.float16 if epi in (oracle.EPI_F16, oracle.EPI_GELU16) else torch.float32
        y0 = torch.randn((T, rows), generator=gen).to(DEV).to(dt)
        ya, yb = y0.clone(), y0.clone()
        g = gate if epi == oracle.EPI_RESID else None
        kiln_amd.linear16(ya, x, w, epi=epi, gate=g, beta=0.25 if epi == oracle.EPI_F32 else 0.0, a2=a2, w2=w2)
        kiln_amd.linear16(yb, x, wp, epi=epi, gate=g, beta=0.25 if epi == oracle.EPI_F32 else 0.0, a2=a2, w2=w2)
        torch.cuda.synchronize()
        assert torch.equal(ya.view(torch.int16 if dt == torch.float16 else torch.int32),
                           yb.view(torch.int16 if dt == torch.float16 else torch.int32)), f"epi {epi}"


def test_linear16_prepare_weight_from_bf16(gpu):
    """bf16 weights are clamped to the fp16 range and rounded to nearest even (the reference's k_bf16_to_f16,
    engine/src/kernels.cu:531-536), then used as the fp16 weight: equal to the oracle on the converted values."""
    T, rows, cols = 64, 128, 64
    gen = torch.Generator().manual_seed(10)
    x = _f16(gen, (T, cols))
    wb = (torch.randn((rows, cols), generator=gen) * 0.3).to(torch.bfloat16)
    wb[0, :4] = torch.tensor([70000.0, -1e6, 65504.0, 1.0009765625], dtype=torch.bfloat16)  # clamp and rounding
    w16 = wb.float().clamp(-65504, 65504).to(torch.float16)
    wp = kiln_amd.linear16_prepare_weight(wb.to(DEV))
    y = torch.zeros((T, rows), device=DEV)
    kiln_amd.linear16(y, x.to(DEV), wp)
    ref = oracle.linear16(_bits(x), _bits(w16), oracle.EPI_F32)
    _check(oracle.EPI_F32, y.cpu().double().numpy(), ref.astype(np.float64), _abs_acc(x, w16), cols)
