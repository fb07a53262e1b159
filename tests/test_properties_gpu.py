"""Size-independent properties of the HIP attention path at the BASELINE configs' full sizes, where the CPU
oracle would take minutes: each property fixes the exact answer (or its relation to another call) without
a reference run. All calls go through the C ABI.

* V = 1 everywhere: the softmax weights sum to one, so every output is 1 (the kernel's row sum adds the same
  fp16-rounded P values the PV product consumes, so the only error is fp32 rounding).
* Linearity in V: attn(Q, K, V1 + V2) = attn(Q, K, V1) + attn(Q, K, V2), to fp16 output rounding.
* Key permutation: permuting the rows of K and V together leaves the output unchanged (the online softmax
  visits the keys in another order), to fp16 output rounding.
* Determinism: two identical calls give bit-identical outputs.
* CFG batching: the batched fused call equals one call per batch item, bit for bit.
* One key (Tk = 1): every softmax weight is exactly 1, so every query row's output is that key's V row, bit for bit
  (fp16 V through an fp32 accumulator back to fp16).
* Identical keys: every score of a row is the same, every weight exactly 1 after the max shift, so the output is
  the mean of the V rows (the row sum counts the keys exactly), to fp16 output rounding.
"""
import numpy as np
import pytest
import torch

import kiln_amd

pytestmark = pytest.mark.gpu
H, D = 16, 128
DEV = "cuda:0"
# fp16 outputs of magnitude <= ~1: one fp16 ulp at 1 is 2^-10; sums of two rounded outputs differ by <= 2 ulp
F16_TOL = 2.5e-3


def _dit_inputs(B, T, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    X = torch.randn(B * T, H * D, generator=g, device=DEV)
    out = []
    for _ in range(3):
        W = (torch.rand(H * D, H * D, generator=g, device=DEV) * 2 - 1) / (H * D) ** 0.5
        out.append((X @ W.T).half())
    return out


def _rope(Hp, Wp):
    c, s = kiln_amd.cosmos_rope_tables(Hp, Wp)
    return c.to(DEV), s.to(DEV)


def _self(q, k, v, B, T, rope, w):
    out = torch.empty_like(q)
    kiln_amd.dit_self_attn(out, q, k, v, B, T, H, w, w, rope)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("Hp,Wp", [(64, 64), (48, 72)])  # config 4 (T=4096) and config 5 (T=3456)
def test_ones_value_gives_ones(gpu, Hp, Wp):
    T, B = Hp * Wp, 2
    print(f"[case] V=1, fused DiT self-attention B={B} T={T}", flush=True)
    q, k, _ = _dit_inputs(B, T, 11)
    v = torch.ones_like(q)
    w = (torch.rand(D, generator=torch.Generator().manual_seed(3)) * 2 + 1).to(torch.bfloat16).to(DEV)
    out = _self(q, k, v, B, T, _rope(Hp, Wp), w).float()
    err = (out - 1).abs().max().item()
    print(f"[parity] V=1: max |out - 1| = {err:.3e}", flush=True)
    assert err <= 1e-3


def test_linearity_in_v(gpu):
    T, B, Hp, Wp = 4096, 2, 64, 64
    print(f"[case] linearity in V, fused DiT self-attention B={B} T={T}", flush=True)
    q, k, v1 = _dit_inputs(B, T, 21)
    v2 = torch.randn(v1.shape, generator=torch.Generator(device=DEV).manual_seed(5), device=DEV).half() * 0.5
    w = torch.ones(D, dtype=torch.bfloat16, device=DEV)
    rope = _rope(Hp, Wp)
    o1 = _self(q, k, v1, B, T, rope, w).float()
    o2 = _self(q, k, v2, B, T, rope, w).float()
    o12 = _self(q, k, (v1.float() + v2.float()).half(), B, T, rope, w).float()
    # v1 + v2 is itself rounded to fp16: bound its effect by the output magnitude of that rounding
    err = (o12 - o1 - o2).abs().max().item()
    scale = max(1.0, o12.abs().max().item())
    print(f"[parity] linearity: max |o(v1+v2) - o(v1) - o(v2)| = {err:.3e} (output scale {scale:.2f})", flush=True)
    assert err <= F16_TOL * scale


def test_key_permutation_invariance(gpu):
    S = 4096
    print(f"[case] key permutation, fp16-in batched attention B=1 T={S}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(31)
    q, k, v = (torch.randn(S, H * D, generator=g, device=DEV).half() for _ in range(3))
    perm = torch.randperm(S, generator=torch.Generator().manual_seed(7)).to(DEV)
    o = torch.empty_like(q)
    op = torch.empty_like(q)
    kiln_amd.attn_f16in(o, q, k, v, 1, S, S, H)
    kiln_amd.attn_f16in(op, q, k[perm].contiguous(), v[perm].contiguous(), 1, S, S, H)
    torch.cuda.synchronize()
    err = (o.float() - op.float()).abs().max().item()
    print(f"[parity] permuted keys: max diff {err:.3e}", flush=True)
    assert err <= F16_TOL


def test_determinism_and_batch_split(gpu):
    T, B, Hp, Wp = 1536, 2, 32, 48  # config 2
    print(f"[case] determinism / per-item split, fused DiT self-attention B={B} T={T}", flush=True)
    q, k, v = _dit_inputs(B, T, 41)
    w = torch.ones(D, dtype=torch.bfloat16, device=DEV)
    rope = _rope(Hp, Wp)
    a = _self(q, k, v, B, T, rope, w)
    b = _self(q, k, v, B, T, rope, w)
    assert torch.equal(a, b), "two identical calls differ"
    for i in range(B):
        sl = slice(i * T, (i + 1) * T)
        one = _self(q[sl].contiguous(), k[sl].contiguous(), v[sl].contiguous(), 1, T, rope, w)
        assert torch.equal(one, a[sl]), f"batch item {i} differs from its single-item call"
    print("[parity] bit-identical repeat and per-item split", flush=True)


def test_cross_attention_nag_full_size_neutral(gpu):
    """Config 5 cross-attention shape (T=3456, L=512, B=2, NAG on item 0): with the negative context equal to
    the positive one, NAG's guidance g = a*s - an*(s-1) equals a, no clamp applies, and the blend returns a;
    so item 0's output must equal the same call without NAG (to fp16 rounding of the blend)."""
    T, B, L = 3456, 2, 512
    print(f"[case] cross-attention + NAG, neutral negative context, T={T} L={L}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(51)
    q = torch.randn(B * T, H * D, generator=g, device=DEV).half()
    w = torch.ones(D, dtype=torch.bfloat16, device=DEV)
    ctx = [kiln_amd.kv_prepare(torch.randn(L, H * D, generator=g, device=DEV).half(),
                               torch.randn(L, H * D, generator=g, device=DEV).half(), H, k_norm_w=w) for _ in range(2)]
    plain = torch.empty_like(q)
    kiln_amd.cross_attn_nag(plain, q, B, T, H, ctx, [L, L], [0, 0], q_norm_w=w)
    nag = torch.empty_like(q)
    neg = torch.empty(T, H * D, dtype=torch.float16, device=DEV)
    kiln_amd.cross_attn_nag(nag, q, B, T, H, ctx, [L, L], [0, 0], q_norm_w=w, kvp_neg=ctx[0], Lk_neg=L, npad_neg=0,
                            out_neg=neg)
    torch.cuda.synchronize()
    assert torch.equal(neg, plain[:T]), "negative attention over the same context differs from item 0"
    assert torch.equal(nag[T:], plain[T:]), "item 1 must not be touched by NAG"
    err = (nag[:T].float() - plain[:T].float()).abs().max().item()
    print(f"[parity] neutral NAG on item 0: max diff {err:.3e}", flush=True)
    assert err <= 1e-3


def test_single_key_returns_its_value_row(gpu):
    B, Tq = 2, 4096
    print(f"[case] Tk=1, fp16-in batched attention B={B} Tq={Tq}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(51)
    q = torch.randn(B * Tq, H * D, generator=g, device=DEV).half()
    k = torch.randn(B, H * D, generator=g, device=DEV).half()
    v = torch.randn(B, H * D, generator=g, device=DEV).half()
    o = torch.empty_like(q)
    kiln_amd.attn_f16in(o, q, k, v, B, Tq, 1, H)
    torch.cuda.synchronize()
    for b in range(B):
        assert torch.equal(o[b * Tq:(b + 1) * Tq], v[b:b + 1].expand(Tq, -1)), f"item {b}: output is not V's one row"
    print("[parity] Tk=1: every output row equals the key's V row", flush=True)


@pytest.mark.parametrize("Tk", [4096, 1000])  # whole 64-key tiles, and a ragged last half tile
def test_identical_keys_give_mean_value(gpu, Tk):
    Tq = 2048
    print(f"[case] identical keys, fp16-in attention Tq={Tq} Tk={Tk}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(61)
    q = torch.randn(Tq, H * D, generator=g, device=DEV).half()
    k = torch.randn(1, H * D, generator=g, device=DEV).half().expand(Tk, -1).contiguous()
    v = torch.randn(Tk, H * D, generator=g, device=DEV).half()
    o = torch.empty_like(q)
    kiln_amd.attn_f16in(o, q, k, v, 1, Tq, Tk, H)
    torch.cuda.synchronize()
    mean = v.double().mean(0, keepdim=True).expand(Tq, -1)
    err = (o.double() - mean).abs().max().item()
    print(f"[parity] identical keys: max |out - mean(V)| = {err:.3e}", flush=True)
    assert err <= 2e-4  # |mean| ~ 0.02-0.1: fp16 rounding of the output (<= 2^-14) and fp32 sums of Tk terms
