"""One DiT block on the fp16-activation path (kiln_amd.dit.block_forward16, composed of the library's entry
points) against a float64 restatement of the reference's block loop (engine/src/dit.cu:458-493).

The restatement rounds to fp16 where the reference's fp16 path stores fp16 (the modulated LayerNorm output,
the attention outputs, the NAG combine, the GELU output) and keeps everything else exact, so the difference
is the accumulated error of the GPU kernels (fp16 attention semantics, fp32 GEMM accumulation, neighbouring
fp16 roundings). Bar on the block output X (values ~N(0,1)): max-abs 1e-2, mean-abs 5e-4.
"""
import numpy as np
import pytest
import torch

import kiln_amd
import oracle
from kiln_amd import dit

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
HD = 128


def _bf16(t):
    return t.to(torch.bfloat16)


def _rms(x, w, H, eps):
    xs = x.view(x.shape[0], H, HD)
    r = torch.rsqrt((xs * xs).mean(-1, keepdim=True) + eps)
    return (xs * r * w.double()).view(x.shape[0], H * HD)


def _rope(x, c, s, H):
    xs = x.view(x.shape[0], H, HD)
    a, b = xs[..., :64], xs[..., 64:]
    c, s = c[:, None, :], s[:, None, :]
    return torch.cat([a * c - b * s, b * c + a * s], -1).reshape(x.shape[0], H * HD)


def _attn(q, k, v, H, npad=0):
    T = q.shape[0]
    qs, ks, vs = (t.view(t.shape[0], H, HD).transpose(0, 1) for t in (q, k, v))
    sc = qs @ ks.transpose(1, 2) / np.sqrt(HD)
    if npad:
        sc = torch.cat([sc, torch.zeros(H, T, npad, dtype=sc.dtype)], -1)
        vs = torch.cat([vs, torch.zeros(H, npad, HD, dtype=vs.dtype)], 1)
    return (torch.softmax(sc, -1) @ vs).transpose(0, 1).reshape(T, H * HD)


def _r16(x):
    return x.to(torch.float16).double()


def _ln16(x, shift, scale, eps):
    m = x.mean(-1, keepdim=True)
    var = ((x - m) ** 2).mean(-1, keepdim=True)
    return _r16((x - m) / torch.sqrt(var + eps) * (1 + scale) + shift)


def test_dit_block_forward16_matches_reference(gpu):
    H, Hp, Wp, B, Dctx, L = 4, 8, 12, 2, 256, 64
    D, F, T, eps = H * HD, 4 * H * HD, Hp * Wp, 1e-6
    g = torch.Generator().manual_seed(31)

    def w16(o, i):
        return (torch.randn(o, i, generator=g) * i ** -0.5).half()

    Wqkv, Wo, Wcq, Wco, W1, W2 = w16(3 * D, D), w16(D, D), w16(D, D), w16(D, D), w16(F, D), w16(D, F)
    Wck, Wcv = torch.randn(D, Dctx, generator=g) * Dctx ** -0.5, torch.randn(D, Dctx, generator=g) * Dctx ** -0.5
    nw = [_bf16(1 + 0.2 * torch.randn(HD, generator=g)) for _ in range(4)]  # sa_qn, sa_kn, ca_qn, ca_kn
    mods = torch.randn(9 * D, generator=g) * 0.3
    X0 = torch.randn(B * T, D, generator=g)
    reals = [40, 64, 33]  # prompt, unconditional, NAG negative: real rows of 64-row contexts
    ctxs = [torch.randn(r, Dctx, generator=g) for r in reals]
    nag = (5.0, 2.5, 0.25)

    blk = dit.Block16(Wqkv.to(DEV), Wo.to(DEV), Wcq.to(DEV), Wco.to(DEV), W1.to(DEV), W2.to(DEV),
                      *[w.to(DEV) for w in nw], ca_k=Wck.to(DEV), ca_v=Wcv.to(DEV))
    kvs = [blk.prepare_context(c.to(DEV), eps) for c in ctxs]
    rc, rs = kiln_amd.cosmos_rope_tables(Hp, Wp)
    ws = dit.Workspace(B, T, D, F, DEV)
    X = X0.to(DEV).clone()
    dit.block_forward16(X, mods.to(DEV), blk, ws, B, T, (rc.to(DEV), rs.to(DEV)),
                        [(kvs[i], reals[i], L - reals[i]) for i in range(B)],
                        nag=(kvs[2], reals[2], L - reals[2]) + nag, eps=eps)
    torch.cuda.synchronize()

    # float64 restatement
    d = lambda t: t.double()  # noqa: E731
    x = d(X0)
    mo, mc, mm = d(mods[:3 * D]), d(mods[3 * D:6 * D]), d(mods[6 * D:])
    n = _ln16(x, mo[:D], mo[D:2 * D], eps)
    qkv = n @ d(Wqkv).T
    a = torch.empty(B * T, D, dtype=torch.float64)
    for b in range(B):
        rows = slice(b * T, (b + 1) * T)
        q = _rope(_rms(qkv[rows, :D], d(nw[0].float()), H, eps), d(rc), d(rs), H)
        k = _rope(_rms(qkv[rows, D:2 * D], d(nw[1].float()), H, eps), d(rc), d(rs), H)
        a[rows] = _r16(_attn(q, k, qkv[rows, 2 * D:], H))
    x = x + mo[2 * D:] * (a @ d(Wo).T)
    n = _ln16(x, mc[:D], mc[D:2 * D], eps)
    qc = _rms(n @ d(Wcq).T, d(nw[2].float()), H, eps)
    kc = [_rms(d(c) @ d(Wck).T, d(nw[3].float()), H, eps) for c in ctxs]
    vc = [d(c) @ d(Wcv).T for c in ctxs]
    for b in range(B):
        rows = slice(b * T, (b + 1) * T)
        a[rows] = _r16(_attn(qc[rows], kc[b], vc[b], H, L - reals[b]))
    an = _r16(_attn(qc[:T], kc[2], vc[2], H, L - reals[2]))
    a[:T] = _r16(torch.from_numpy(oracle.nag(a[:T].numpy(), an.numpy(), *nag)).double())
    x = x + mc[2 * D:] * (a @ d(Wco).T)
    n = _ln16(x, mm[:D], mm[D:2 * D], eps)
    h = n @ d(W1).T
    h = _r16(0.5 * h * (1 + torch.erf(h / np.sqrt(2))))
    x = x + mm[2 * D:] * (h @ d(W2).T)

    err = (X.cpu().double() - x).abs()
    assert torch.isfinite(X).all()
    assert err.max().item() <= 1e-2 and err.mean().item() <= 5e-4, (err.max().item(), err.mean().item())
