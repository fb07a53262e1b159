"""Randomised (but fixed-seed, deterministic) parity sweep over the flash path's entry points.

Every case draws a route through the C ABI, a head count, ragged query/key counts, npad zero keys, padded
row strides and a column offset of the head block, and compares with the CPU oracle (double-accumulation
softmax attention) at the BASELINE bar (max-abs 2e-3, mean-abs 2e-4). Inputs are N(0, 1).
Routes:
  f32out  attention()   (engine/src/gpu.h:149-153): fp32 Q/K/V, fp32 out, some cases causal
  f16out  attention16() (engine/src/gpu.h:155-156): fp32 Q/K/V, fp16 out
  f16in   kiln_attn_fwd_f16in: fp16 Q/K/V, B batch items, fp16 or fp32 out
  dit     kiln_dit_self_attn_fused: QK-RMSNorm (bf16 weights) + Cosmos RoPE + attention, B items, fp16 or fp32 out
"""
import numpy as np
import pytest
import torch

import kiln_amd
import oracle
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu
D = 128
DEV = "cuda:0"


def _cases(n=24, seed=2024):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        route = ["f32out", "f16out", "f16in", "dit"][i % 4]
        c = dict(route=route, H=int(rng.choice([1, 2, 3, 5, 16])), pad=[int(rng.choice([0, 8, 24])) for _ in range(4)],
                 off=int(rng.choice([0, 8])), seed=1000 + i)
        if route == "dit":
            c.update(Hp=int(rng.integers(2, 20)), Wp=int(rng.integers(2, 24)), B=int(rng.integers(1, 4)),
                     f32=bool(rng.integers(0, 2)), out32=bool(rng.integers(0, 2)))
        else:
            c.update(Tq=int(rng.integers(1, 600)), Tk=int(rng.integers(1, 800)),
                     npad=int(rng.choice([0, 0, int(rng.integers(1, 300))])), B=int(rng.integers(1, 5)),
                     out32=bool(rng.integers(0, 2)), causal=route == "f32out" and (i // 4) % 3 == 0)
        out.append(c)
    return out


CASES = _cases()


def _split_cases(n=8, seed=77):
    """Few heads and queries against long key sequences: grids under a third of the workgroup slots, so the
    launch splits every query tile's keys into ranges and merges the partials (fp32/fp16 drop-ins and the
    batched fp16 entry point with the library's workspace)."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        route = ["f32out", "f16out", "f16in"][i % 3]
        out.append(dict(route=route, H=int(rng.choice([1, 2])), pad=[int(rng.choice([0, 8, 24])) for _ in range(4)],
                        off=int(rng.choice([0, 8])), seed=5000 + i, Tq=int(rng.integers(1, 400)),
                        Tk=int(rng.integers(1500, 5000)), npad=int(rng.choice([0, int(rng.integers(1, 300))])),
                        B=int(rng.integers(1, 3)), out32=bool(rng.integers(0, 2)), causal=False))
    return out


SPLIT_CASES = _split_cases()


def _wide_cases(n=8, seed=4242):
    """Grids of 256-row query tiles that fill whole rounds of a 256-CU part (tiles x H x B = 256 or 512), which
    run the 8-wave kernel: every route, ragged query and key counts, npad, padded strides and offsets."""
    rng = np.random.default_rng(seed)
    shapes = [(16, 1, 16), (16, 2, 8), (32, 1, 8), (8, 4, 8), (16, 4, 4), (16, 2, 16)]  # (H, B, query tiles)
    out = []
    for i in range(n):
        route = ["f32out", "f16out", "f16in", "dit"][i % 4]
        H, B, nt = shapes[int(rng.integers(0, len(shapes)))]
        if route in ("f32out", "f16out"):  # single-item routes: H x tiles must fill the rounds alone
            H, B, nt = (16, 1, 16) if i % 2 == 0 else (32, 1, 8)
        if route == "dit":  # the oracle's full-row reference: keep T x T x B small
            H, B, nt = [(16, 4, 4), (16, 2, 8), (8, 4, 8)][i % 3]
        c = dict(route=route, H=H, B=B, pad=[int(rng.choice([0, 8, 24])) for _ in range(4)],
                 off=int(rng.choice([0, 8])), seed=7000 + i)
        lo, hi = 256 * (nt - 1) + 1, 256 * nt
        if route == "dit":
            Wp = int(rng.integers(24, 48))
            Hp = -(-lo // Wp)  # smallest Hp with Hp * Wp in the tile range
            if Hp * Wp > hi:
                Hp, Wp = nt * 8, 32  # T = 256 nt
            c.update(Hp=Hp, Wp=Wp, f32=bool(rng.integers(0, 2)), out32=bool(rng.integers(0, 2)))
        else:
            c.update(Tq=int(rng.integers(lo, hi + 1)), Tk=int(rng.integers(1, 1200)),
                     npad=int(rng.choice([0, int(rng.integers(1, 300))])), out32=bool(rng.integers(0, 2)),
                     causal=False)
        out.append(c)
    return out


WIDE_CASES = _wide_cases()


def _strided(rows, H, pad, off, dtype, data):
    """[rows, H*D] view of a [rows, off + H*D + pad] buffer (row stride = off + H*D + pad), holding data."""
    buf = torch.zeros(rows, off + H * D + pad, dtype=dtype, device=DEV)
    view = buf[:, off:off + H * D]
    if data is not None:
        view.copy_(data.to(dtype))
    return view


@pytest.mark.parametrize("idx", range(len(CASES)))
def test_random_shapes(gpu, idx):
    _run_case(CASES[idx], idx)


@pytest.mark.parametrize("idx", range(len(SPLIT_CASES)))
def test_random_split_shapes(gpu, idx):
    _run_case(SPLIT_CASES[idx], 100 + idx)


@pytest.mark.parametrize("idx", range(len(WIDE_CASES)))
def test_random_eight_wave_shapes(gpu, idx):
    _run_case(WIDE_CASES[idx], 200 + idx)


def _run_case(c, idx):
    H, pad, off = c["H"], c["pad"], c["off"]
    g = torch.Generator().manual_seed(c["seed"])
    print(f"[random] case {idx}: {c}", flush=True)
    if c["route"] == "dit":
        Hp, Wp, B = c["Hp"], c["Wp"], c["B"]
        T = Hp * Wp
        dt = torch.float32 if c["f32"] else torch.float16
        q, k, v = (torch.randn(B * T, H * D, generator=g).to(dt).float() for _ in range(3))
        qw = (torch.rand(D, generator=g) + 0.5).to(torch.bfloat16)
        kw = (torch.rand(D, generator=g) + 0.5).to(torch.bfloat16)
        cos, sin = oracle.cosmos_rope(Hp, Wp)
        qwb = qw.view(torch.int16).numpy().view(np.uint16)
        kwb = kw.view(torch.int16).numpy().view(np.uint16)
        refs = []
        for b in range(B):
            sl = slice(b * T, (b + 1) * T)
            qn = oracle.rope_half(oracle.rmsnorm_rows(q[sl].numpy(), qwb).reshape(T, H * D), H, cos, sin)
            kn = oracle.rope_half(oracle.rmsnorm_rows(k[sl].numpy(), kwb).reshape(T, H * D), H, cos, sin)
            refs.append(oracle.attn_f64(qn, kn, v[sl].numpy(), H))
        ld = off + H * D + pad[0]  # the fused entry point takes one row stride for Q, K and V
        qd, kd, vd = (_strided(B * T, H, pad[0], off, dt, t) for t in (q, k, v))
        assert qd.stride(0) == ld
        out = _strided(B * T, H, pad[3], off, torch.float32 if c["out32"] else torch.float16, None)
        rope = (torch.from_numpy(cos).to(DEV), torch.from_numpy(sin).to(DEV))
        kiln_amd.dit_self_attn(out, qd, kd, vd, B, T, H, qw.to(DEV), kw.to(DEV), rope)
        torch.cuda.synchronize()
        o = out.float().cpu().numpy()
        for b in range(B):
            assert_close(o[b * T:(b + 1) * T], refs[b], f"case {idx} dit b={b}")
        return

    Tq, Tk, npad = c["Tq"], c["Tk"], c["npad"]
    if c["route"] == "f16in":
        B = c["B"]
        q, k, v = (torch.randn(B * T_, H * D, generator=g).half().float() for T_ in (Tq, Tk, Tk))
        odt = torch.float32 if c["out32"] else torch.float16
        qd = _strided(B * Tq, H, pad[0], off, torch.float16, q)
        kd = _strided(B * Tk, H, pad[1], off, torch.float16, k)
        vd = _strided(B * Tk, H, pad[2], off, torch.float16, v)
        out = _strided(B * Tq, H, pad[3], off, odt, None)
        kiln_amd.attn_f16in(out, qd, kd, vd, B, Tq, Tk, H, npad=npad)
        torch.cuda.synchronize()
        o = out.float().cpu().numpy()
        for b in range(B):
            ref = oracle.attn_f64(q[b * Tq:(b + 1) * Tq].numpy(), k[b * Tk:(b + 1) * Tk].numpy(),
                                  v[b * Tk:(b + 1) * Tk].numpy(), H, npad=npad)
            assert_close(o[b * Tq:(b + 1) * Tq], ref, f"case {idx} f16in b={b}")
        return

    q, k, v = (torch.randn(T_, H * D, generator=g) for T_ in (Tq, Tk, Tk))
    ref = oracle.attn_f64(q.numpy(), k.numpy(), v.numpy(), H, npad=npad, causal=c["causal"])
    qd = _strided(Tq, H, pad[0], off, torch.float32, q)
    kd = _strided(Tk, H, pad[1], off, torch.float32, k)
    vd = _strided(Tk, H, pad[2], off, torch.float32, v)
    if c["route"] == "f32out":
        out = _strided(Tq, H, pad[3], off, torch.float32, None)
        kiln_amd.attention(out, qd, kd, vd, Tq, Tk, H, D, causal=c["causal"], npad=npad)
    else:
        out = _strided(Tq, H, pad[3], off, torch.float16, None)
        kiln_amd.attention16(out, qd, kd, vd, Tq, Tk, H, D, npad=npad)
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy(), ref, f"case {idx} {c['route']}")


# Output row stride / base alignment -> store path of the attention epilogue: 16-byte aligned rows are staged
# through LDS and stored as whole rows; 8-byte aligned fp16 rows take 4-element stores; anything else element
# pairs.
ALIGN_CASES = [(torch.float16, 0, 0), (torch.float16, 4, 0), (torch.float16, 2, 6), (torch.float32, 0, 4),
               (torch.float32, 2, 0), (torch.float32, 4, 2)]


@pytest.mark.parametrize("odt,off,pad", ALIGN_CASES)
def test_output_alignment_paths(gpu, odt, off, pad):
    H, B, Tq, Tk = 3, 2, 300, 257
    g = torch.Generator().manual_seed(31 + off + pad)
    print(f"[random] output alignment {odt} off={off} pad={pad}", flush=True)
    q, k, v = (torch.randn(B * T_, H * D, generator=g).half().float() for T_ in (Tq, Tk, Tk))
    qd = _strided(B * Tq, H, 8, 0, torch.float16, q)
    kd = _strided(B * Tk, H, 0, 0, torch.float16, k)
    vd = _strided(B * Tk, H, 24, 0, torch.float16, v)
    out = _strided(B * Tq, H, pad, off, odt, None)
    kiln_amd.attn_f16in(out, qd, kd, vd, B, Tq, Tk, H)
    torch.cuda.synchronize()
    o = out.float().cpu().numpy()
    for b in range(B):
        ref = oracle.attn_f64(q[b * Tq:(b + 1) * Tq].numpy(), k[b * Tk:(b + 1) * Tk].numpy(),
                              v[b * Tk:(b + 1) * Tk].numpy(), H)
        assert_close(o[b * Tq:(b + 1) * Tq], ref, f"alignment {odt} off={off} pad={pad} b={b}")
