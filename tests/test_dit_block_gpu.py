"""The DiT through the C++ step driver (libkiln_dit.so, kiln_amd.dit.Dit): one block on the fp16-activation path
against a float64 restatement of the reference's block loop (engine/src/dit.cu:458-493), the whole forward, the
step cache and the fp32 block; plus the DiT's auxiliary kernels.

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


H, Hp, Wp, B, DCTX, L = 4, 8, 12, 2, 256, 64
D, F, T, EPS = H * HD, 4 * H * HD, Hp * Wp, 1e-6
REALS = [40, 64, 33]  # prompt, unconditional, NAG negative: real rows of 64-row contexts
NAG = (5.0, 2.5, 0.25)


def _bf16w(g, o, i, scale=None):
    return _bf16(torch.randn(o, i, generator=g) * (scale if scale is not None else i ** -0.5))


def _block_weights(g):
    """Random bf16 weights of one block [out, in] (host), as a checkpoint holds them."""
    w = dict(sa_q=_bf16w(g, D, D), sa_k=_bf16w(g, D, D), sa_v=_bf16w(g, D, D), sa_o=_bf16w(g, D, D),
             ca_q=_bf16w(g, D, D), ca_o=_bf16w(g, D, D), ca_k=_bf16w(g, D, DCTX), ca_v=_bf16w(g, D, DCTX),
             mlp1=_bf16w(g, F, D), mlp2=_bf16w(g, D, F))
    for n in ("sa_qn", "sa_kn", "ca_qn", "ca_kn"):
        w[n] = _bf16(1 + 0.2 * torch.randn(HD, generator=g))
    w["mod"] = [_bf16w(g, 256, D), _bf16w(g, 3 * D, 256), _bf16w(g, 256, D), _bf16w(g, 3 * D, 256),
                _bf16w(g, 256, D), _bf16w(g, 3 * D, 256)]
    return w


def _make_dit(g, nblocks):
    """A Dit of nblocks random blocks (H = 4, D = 512, F = 2048, 256-wide contexts) and random step weights."""
    d = dit.Dit(nblocks, H, ctx_dim=DCTX, mlp=F, eps=EPS)
    ws = []
    for i in range(nblocks):
        w = _block_weights(g)
        d.set_block(i, **{k: (v.to(DEV) if torch.is_tensor(v) else [m.to(DEV) for m in v]) for k, v in w.items()})
        ws.append(w)
    sw = dict(t_lin1=_bf16w(g, D, D), t_lin2=_bf16w(g, 3 * D, D), t_norm=_bf16(1 + 0.1 * torch.randn(D, generator=g)),
              final_mod1=_bf16w(g, 256, D), final_mod2=_bf16w(g, 2 * D, 256), x_embed=_bf16w(g, D, 68, 68 ** -0.5),
              final_lin=_bf16w(g, 64, D))
    d.set_step_weights(**{k: v.to(DEV) for k, v in sw.items()})
    return d, ws, sw


def _h(w):
    """A linear16 weight as the fp16 path uses it: bf16 converted to fp16 at load (weight_to_f16)."""
    return w.float().half().double()


def _ctx_kv(w, c):
    """Dit::cache_context (engine/src/dit.cu:217-234): K = rmsnorm(ctx W_k^T; ca_kn), V = ctx W_v^T."""
    k = _rms(c.double() @ w["ca_k"].float().double().T, w["ca_kn"].float().double(), H, EPS)
    return k, c.double() @ w["ca_v"].float().double().T


def _ref_block(x, mods, w, ctxs, rc, rs):
    """float64 restatement of one block (engine/src/dit.cu:458-493), fp16 rounding where the fp16 path stores."""
    d = lambda t: t.double()  # noqa: E731
    nw = {k: d(w[k].float()) for k in ("sa_qn", "sa_kn", "ca_qn")}
    mo, mc, mm = d(mods[:3 * D]), d(mods[3 * D:6 * D]), d(mods[6 * D:])
    n = _ln16(x, mo[:D], mo[D:2 * D], EPS)
    a = torch.empty(B * T, D, dtype=torch.float64)
    for b in range(B):
        rows = slice(b * T, (b + 1) * T)
        q = _rope(_rms(n[rows] @ _h(w["sa_q"]).T, nw["sa_qn"], H, EPS), d(rc), d(rs), H)
        k = _rope(_rms(n[rows] @ _h(w["sa_k"]).T, nw["sa_kn"], H, EPS), d(rc), d(rs), H)
        a[rows] = _r16(_attn(q, k, n[rows] @ _h(w["sa_v"]).T, H))
    x = x + mo[2 * D:] * (a @ _h(w["sa_o"]).T)
    n = _ln16(x, mc[:D], mc[D:2 * D], EPS)
    qc = _rms(n @ _h(w["ca_q"]).T, nw["ca_qn"], H, EPS)
    kv = [_ctx_kv(w, c) for c in ctxs]
    for b in range(B):
        rows = slice(b * T, (b + 1) * T)
        a[rows] = _r16(_attn(qc[rows], kv[b][0], kv[b][1], H, L - REALS[b]))
    an = _r16(_attn(qc[:T], kv[2][0], kv[2][1], H, L - REALS[2]))
    a[:T] = _r16(torch.from_numpy(oracle.nag(a[:T].numpy(), an.numpy(), *NAG)).double())
    x = x + mc[2 * D:] * (a @ _h(w["ca_o"]).T)
    n = _ln16(x, mm[:D], mm[D:2 * D], EPS)
    h = n @ _h(w["mlp1"]).T
    h = _r16(0.5 * h * (1 + torch.erf(h / np.sqrt(2))))
    return x + mm[2 * D:] * (h @ _h(w["mlp2"]).T)


def test_dit_block_forward16_matches_reference(gpu):
    """One block (Dit::run_block, fp16 path) with random modulation and contexts cached by the driver."""
    g = torch.Generator().manual_seed(31)
    d, ws, _ = _make_dit(g, 1)
    mods = torch.randn(9 * D, generator=g) * 0.3
    X0 = torch.randn(B * T, D, generator=g)
    ctxs = [torch.randn(r, DCTX, generator=g) for r in REALS]
    cc = [d.cache_context(c.to(DEV), length=L) for c in ctxs]
    rc, rs = kiln_amd.cosmos_rope_tables(Hp, Wp)
    X = X0.to(DEV).clone()
    d.run_block(0, X, mods.to(DEV), Hp, Wp, cc[:B], nag=dit.Nag(cc[2], *NAG))
    torch.cuda.synchronize()
    x = _ref_block(X0.double(), mods, ws[0], ctxs, rc, rs)
    err = (X.cpu().double() - x).abs()
    assert torch.isfinite(X).all()
    assert err.max().item() <= 1e-2 and err.mean().item() <= 5e-4, (err.max().item(), err.mean().item())


def _sinusoid(t):
    """The timestep sinusoid of Dit::step_tables (engine/src/dit.cu:246-251) in float32: cos(t e_i), sin(t e_i),
    e_i = exp(-i ln(10000) / (D/2))."""
    i = np.arange(D // 2, dtype=np.float32)
    e = np.exp(i * np.float32(-np.log(np.float32(10000.0))) / np.float32(D // 2)).astype(np.float32)
    te = (np.float32(t) * e).astype(np.float32)
    return np.concatenate([np.cos(te), np.sin(te)]).astype(np.float32)


def _ref_forward(t, ws, sw, latent, ctxs, rc, rs, Hl, Wl):
    d = lambda a: a.double() if torch.is_tensor(a) else torch.from_numpy(a).double()  # noqa: E731
    bw = lambda a: d(a.float())  # noqa: E731
    silu = lambda v: v / (1 + torch.exp(-v))  # noqa: E731
    s = d(_sinusoid(t))
    lora = bw(sw["t_lin2"]) @ silu(bw(sw["t_lin1"]) @ s)
    temb = silu(s / torch.sqrt((s * s).mean() + EPS) * bw(sw["t_norm"]))
    tok = d(oracle.patchify(latent.numpy()))
    x = (tok @ bw(sw["x_embed"]).T).repeat(B, 1)
    for w in ws:
        mods = torch.cat([bw(w["mod"][2 * j + 1]) @ (bw(w["mod"][2 * j]) @ temb) + lora for j in range(3)])
        x = _ref_block(x, mods.float(), w, ctxs, rc, rs)
    fmod = bw(sw["final_mod2"]) @ (bw(sw["final_mod1"]) @ temb) + lora[:2 * D]
    m = x.mean(-1, keepdim=True)
    var = ((x - m) ** 2).mean(-1, keepdim=True)
    n = (x - m) / torch.sqrt(var + EPS) * (1 + fmod[D:]) + fmod[:D]
    y = n @ bw(sw["final_lin"]).T
    return [oracle.unpatchify(y[b * T:(b + 1) * T].float().numpy(), Hl, Wl).astype(np.float64) for b in range(B)]


def test_dit_forward16_two_blocks_matches_reference(gpu):
    """Dit::forward_batch on the fp16 path (engine/src/dit.cu:357-546) with two blocks, through the C++ driver:
    step tables (timestep sinusoid, t_embedder MLP, adaLN modulation matvecs), patch embedding, the blocks, the
    final modulated LayerNorm + linear and unpatchify, against a float64 restatement. Bar on the output latents
    (~N(0,1)): max-abs 2e-2, mean-abs 1e-3."""
    g = torch.Generator().manual_seed(32)
    Hl, Wl, t = 2 * Hp, 2 * Wp, 0.73
    d, ws, sw = _make_dit(g, 2)
    ctxs = [torch.randn(r, DCTX, generator=g) for r in REALS]
    cc = [d.cache_context(c.to(DEV), length=L) for c in ctxs]
    latent = torch.randn(16, Hl, Wl, generator=g)
    rc, rs = kiln_amd.cosmos_rope_tables(Hp, Wp)
    outs = [torch.empty(16, Hl, Wl, device=DEV) for _ in range(B)]
    d.forward(outs, latent.to(DEV), t, cc[:B], nag=dit.Nag(cc[2], *NAG))
    torch.cuda.synchronize()
    refs = _ref_forward(t, ws, sw, latent, ctxs, rc, rs, Hl, Wl)
    for b in range(B):
        err = np.abs(outs[b].cpu().double().numpy() - refs[b])
        assert np.isfinite(err).all()
        assert err.max() <= 2e-2 and err.mean() <= 1e-3, (b, err.max(), err.mean())


def test_dit_forward_odd_latent_pads_circularly(gpu):
    """An odd latent side runs on the circularly padded 2x2 patch grid and is cropped back (engine/src/dit.cu:
    359-371): the result equals the top-left crop of the forward of the padded latent."""
    g = torch.Generator().manual_seed(37)
    d, _, _ = _make_dit(g, 1)
    cc = [d.cache_context(torch.randn(r, DCTX, generator=g).to(DEV), length=L) for r in REALS[:B]]
    Hl, Wl = 2 * Hp - 1, 2 * Wp - 1
    lat = torch.randn(16, Hl, Wl, generator=g).to(DEV)
    padded = torch.cat([lat, lat[:, :1]], 1)
    padded = torch.cat([padded, padded[:, :, :1]], 2).contiguous()
    o_odd = [torch.empty(16, Hl, Wl, device=DEV) for _ in range(B)]
    o_pad = [torch.empty(16, Hl + 1, Wl + 1, device=DEV) for _ in range(B)]
    d.forward(o_odd, lat, 0.5, cc)
    d.forward(o_pad, padded, 0.5, cc)
    torch.cuda.synchronize()
    for a, b_ in zip(o_odd, o_pad):
        assert torch.equal(a, b_[:, :Hl, :Wl].contiguous())


@pytest.mark.parametrize("rows,cols", [(256, 2048), (6144, 256), (37, 100)])
def test_matvec_bf16(gpu, rows, cols):
    g = torch.Generator().manual_seed(rows + cols)
    W = _bf16w(g, rows, cols, 1.0)
    x, add = torch.randn(cols, generator=g), torch.randn(rows, generator=g)
    y = torch.empty(rows, device=DEV)
    kiln_amd.matvec(y, W.to(DEV), x.to(DEV), add=add.to(DEV))
    ref = oracle.matvec_bf16(W.view(torch.int16).numpy().view(np.uint16), x.numpy(), add.numpy())
    bar = np.sqrt(cols) * 2.0 ** -21 * (np.abs(W.float().numpy()) @ np.abs(x.numpy())) + 1e-6
    assert (np.abs(y.cpu().numpy() - ref) <= bar).all()


def test_linear_f32_patchify_silu_cfg(gpu):
    g = torch.Generator().manual_seed(5)
    Hl, Wl = 14, 22
    lat = torch.randn(16, Hl, Wl, generator=g)
    tok = torch.empty((Hl // 2) * (Wl // 2), 68, device=DEV)
    kiln_amd.patchify(tok, lat.to(DEV))
    np.testing.assert_array_equal(tok.cpu().numpy(), oracle.patchify(lat.numpy()))
    y = torch.randn(tok.shape[0], 80, generator=g)  # row stride 80 >= 64
    out = torch.full((16, Hl, Wl), float("nan"), device=DEV)
    kiln_amd.unpatchify(out, y.to(DEV)[:, :64])
    np.testing.assert_array_equal(out.cpu().numpy(), oracle.unpatchify(y[:, :64].contiguous().numpy(), Hl, Wl))
    # (77, 2048, 68) and (300, 64, 2048) take the one-wave kernel; the others the LDS-tiled one (ragged T and rows)
    for T_, rows, cols in [(77, 2048, 68), (300, 64, 2048), (300, 200, 96), (513, 384, 512)]:
        x = torch.randn(T_, cols, generator=g)
        W = _bf16w(g, rows, cols)
        yy = torch.empty(T_, rows, device=DEV)
        kiln_amd.linear_f32(yy, x.to(DEV), W.to(DEV))
        ref = oracle.linear_f32(x.numpy(), W.view(torch.int16).numpy().view(np.uint16))
        bar = np.sqrt(cols) * 2.0 ** -21 * (np.abs(x.numpy()) @ np.abs(W.float().numpy()).T) + 1e-6
        assert (np.abs(yy.cpu().numpy() - ref) <= bar).all()
    v = torch.randn(1000, generator=g) * 4
    sv = torch.empty(1000, device=DEV)
    kiln_amd.silu(sv, v.to(DEV))
    ref = (v.double() * torch.special.expit(v.double())).numpy()
    np.testing.assert_allclose(sv.cpu().double().numpy(), ref, rtol=2e-6, atol=1e-7)
    a, b = torch.randn(999, generator=g), torch.randn(999, generator=g)
    ad = a.to(DEV)
    kiln_amd.cfg_combine(ad, b.to(DEV), 4.5)
    np.testing.assert_allclose(ad.cpu().numpy(), (b.double() + 4.5 * (a.double() - b.double())).numpy(), rtol=1e-6,
                               atol=1e-6)


def test_matvec_bf16_grouped(gpu):
    """The grouped form (the adaLN second layers of all blocks in one launch) equals per-group matvecs."""
    g = torch.Generator().manual_seed(77)
    G_, rows, cols = 6, 384, 256
    W = _bf16w(g, G_ * rows, cols, 1.0).view(G_, rows, cols)
    x, add = torch.randn(G_, cols, generator=g), torch.randn(rows, generator=g)
    y = torch.empty(G_, rows, device=DEV)
    kiln_amd.matvec_grouped(y, W.to(DEV), x.to(DEV), add=add.to(DEV))
    Wb = W.view(torch.int16).numpy().view(np.uint16)
    for i in range(G_):
        ref = oracle.matvec_bf16(Wb[i], x[i].numpy(), add.numpy())
        bar = np.sqrt(cols) * 2.0 ** -21 * (np.abs(W[i].float().numpy()) @ np.abs(x[i].numpy())) + 1e-6
        assert (np.abs(y[i].cpu().numpy() - ref) <= bar).all()


def test_step_cache_skip_reuses_residual(gpu):
    """First-block step cache (engine/src/dit.cu:404-433, 532-536) in the C++ driver: a second forward whose
    block-0 residual did not move skips blocks 1..N-1 and returns the same latents (block-0 output + the cached
    residual); with allow off it runs in full; the relative-L1 and difference kernels against numpy."""
    g = torch.Generator().manual_seed(33)
    d, _, _ = _make_dit(g, 3)
    cc = [d.cache_context(torch.randn(r, DCTX, generator=g).to(DEV), length=L) for r in REALS[:B]]
    latent = torch.randn(16, 2 * Hp, 2 * Wp, generator=g).to(DEV)
    sc = dit.StepCache(0.05)
    sc.allow = True
    o1 = [torch.empty_like(latent) for _ in range(B)]
    d.forward(o1, latent, 0.4, cc, cache=sc)
    assert not sc.skipped and sc.valid
    o2 = [torch.empty_like(latent) for _ in range(B)]
    d.forward(o2, latent, 0.4, cc, cache=sc)
    assert sc.skipped and sc.last_change == 0.0
    for a, b in zip(o1, o2):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)
    sc.allow = False
    o3 = [torch.empty_like(latent) for _ in range(B)]
    d.forward(o3, latent, 0.4, cc, cache=sc)
    assert not sc.skipped
    for a, b in zip(o1, o3):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)
    a, b = torch.randn(100003, generator=g), torch.randn(100003, generator=g)
    acc = torch.empty(2, device=DEV)
    kiln_amd.rel_l1(a.to(DEV), b.to(DEV), acc)
    ref = [np.abs(a.double().numpy() - b.double().numpy()).sum(), np.abs(b.double().numpy()).sum()]
    np.testing.assert_allclose(acc.cpu().double().numpy(), ref, rtol=1e-5)
    y = torch.empty(100003, device=DEV)
    kiln_amd.sub(y, a.to(DEV), b.to(DEV))
    np.testing.assert_array_equal(y.cpu().numpy(), (a - b).numpy())


@pytest.mark.parametrize("Hh,Hp_,Wp_,Bb", [(4, 8, 12, 2), (2, 10, 10, 3), (16, 48, 72, 2), (16, 32, 60, 2)])
def test_dit_self_attn_x16_fused_projection(gpu, Hh, Hp_, Wp_, Bb):
    """kiln_dit_self_attn_x16 (QKV GEMM whose epilogue does QK-RMSNorm, RoPE and the K/V preparation) against
    the float64 statement of dit.cu:460-469 on sampled rows (BASELINE bar: max-abs 2e-3, mean-abs 2e-4), and
    against the unfused path (linear16 F32 + kiln_dit_self_attn_fused) on every output. T = 100 has a partial
    last key tile; T = 3456 x 16 heads is config 5's shape; T = 1920 x 16 heads x 2 items gives 256 query tiles
    of 256 rows, which on a 256-CU part selects the 8-wave attention kernel for both paths."""
    Dd, Tt = Hh * HD, Hp_ * Wp_
    g = torch.Generator().manual_seed(34 + Hh)
    x = (torch.randn(Bb * Tt, Dd, generator=g)).half()
    wqkv = (torch.randn(3 * Dd, Dd, generator=g) * Dd ** -0.5).half()
    qn, kn = (_bf16(1 + 0.2 * torch.randn(HD, generator=g)) for _ in range(2))
    rc, rs = kiln_amd.cosmos_rope_tables(Hp_, Wp_)
    rope = (rc.to(DEV), rs.to(DEV))
    wp = kiln_amd.linear16_prepare_weight(wqkv.to(DEV))
    out = torch.empty(Bb * Tt, Dd, dtype=torch.float16, device=DEV)
    kiln_amd.dit_self_attn_x16(out, x.to(DEV), wp, Bb, Tt, Hh, qn.to(DEV), kn.to(DEV), rope)
    qkv = torch.empty(Bb * Tt, 3 * Dd, device=DEV)
    kiln_amd.linear16(qkv, x.to(DEV), wp)
    ref_u = torch.empty_like(out)
    kiln_amd.dit_self_attn(ref_u, qkv[:, :Dd], qkv[:, Dd:2 * Dd], qkv[:, 2 * Dd:], Bb, Tt, Hh, qn.to(DEV), kn.to(DEV),
                           rope)
    torch.cuda.synchronize()
    du = (out.float() - ref_u.float()).abs()
    assert du.max().item() <= 2e-3 and du.mean().item() <= 1e-4, (du.max().item(), du.mean().item())
    # float64 statement on sampled query rows of every item
    qkv64 = x.double() @ wqkv.double().T
    sel = torch.randperm(Tt, generator=g)[:64]
    errs = []
    for b in range(Bb):
        rows = slice(b * Tt, (b + 1) * Tt)
        q = _rope(_rms(qkv64[rows, :Dd], qn.float().double(), Hh, EPS), rc.double(), rs.double(), Hh)
        k = _rope(_rms(qkv64[rows, Dd:2 * Dd], kn.float().double(), Hh, EPS), rc.double(), rs.double(), Hh)
        ref = _attn(q[sel], k, qkv64[rows, 2 * Dd:], Hh)
        errs.append((out[b * Tt:(b + 1) * Tt][sel.to(DEV)].cpu().double() - ref).abs())
    e = torch.cat(errs)
    assert e.max().item() <= 2e-3 and e.mean().item() <= 2e-4, (e.max().item(), e.mean().item())


def test_dit_cross_attn_x16_fused_projection(gpu):
    """kiln_dit_cross_attn_x16 (cross-Q GEMM with the Q RMSNorm in its epilogue, then cross-attention + NAG)
    against the unfused path (linear16 F32 + kiln_cross_attn_nag) on the same inputs."""
    g = torch.Generator().manual_seed(35)
    x = torch.randn(B * T, D, generator=g).half().to(DEV)
    wq = (torch.randn(D, D, generator=g) * D ** -0.5).half().to(DEV)
    qn, kn = (_bf16(1 + 0.2 * torch.randn(HD, generator=g)).to(DEV) for _ in range(2))
    ctxs = [torch.randn(r, D, generator=g).to(DEV) for r in REALS]
    kvs = [kiln_amd.kv_prepare(c, c * 0.5, H, k_norm_w=kn) for c in ctxs]
    wp = kiln_amd.linear16_prepare_weight(wq)
    out, neg = (torch.empty(n, D, dtype=torch.float16, device=DEV) for n in (B * T, T))
    args = dict(kvp_neg=kvs[2], Lk_neg=REALS[2], npad_neg=L - REALS[2], scale=5.0, tau=2.5, alpha=0.25)
    kiln_amd.dit_cross_attn_x16(out, x, wp, B, T, H, kvs[:B], REALS[:B], [L - r for r in REALS[:B]], qn,
                                out_neg=neg, **args)
    q = torch.empty(B * T, D, device=DEV)
    kiln_amd.linear16(q, x, wp)
    ref, neg2 = torch.empty_like(out), torch.empty_like(neg)
    kiln_amd.cross_attn_nag(ref, q, B, T, H, kvs[:B], REALS[:B], [L - r for r in REALS[:B]], q_norm_w=qn,
                            out_neg=neg2, **args)
    torch.cuda.synchronize()
    d = (out.float() - ref.float()).abs()
    assert torch.isfinite(out.float()).all()
    assert d.max().item() <= 2e-3 and d.mean().item() <= 1e-4, (d.max().item(), d.mean().item())


def test_dit_block_forward32_matches_reference(gpu):
    """The fp32 branch of the block (engine/src/dit.cu:495-530: fp32 linears with bf16 weights, exact fp32
    attention, fp32 GELU), Dit::run_block(fp32=True), against the float64 restatement without fp16 roundings:
    max-abs 1e-3, mean-abs 5e-5."""
    g = torch.Generator().manual_seed(36)
    d_, ws, _ = _make_dit(g, 1)
    w = ws[0]
    mods = torch.randn(9 * D, generator=g) * 0.3
    X0 = torch.randn(B * T, D, generator=g)
    ctxs = [torch.randn(r, DCTX, generator=g) for r in REALS]
    cc = [d_.cache_context(c.to(DEV), length=L, fp32=True) for c in ctxs]
    rc, rs = kiln_amd.cosmos_rope_tables(Hp, Wp)
    X = X0.to(DEV).clone()
    d_.run_block(0, X, mods.to(DEV), Hp, Wp, cc[:B], nag=dit.Nag(cc[2], *NAG), fp32=True)
    torch.cuda.synchronize()
    d = lambda t: t.double()  # noqa: E731
    bf = lambda t: t.float().double()  # noqa: E731
    x = X0.double()
    mo, mc, mm = d(mods[:3 * D]), d(mods[3 * D:6 * D]), d(mods[6 * D:])

    def ln(x, sh, sc):
        m = x.mean(-1, keepdim=True)
        return (x - m) / torch.sqrt(((x - m) ** 2).mean(-1, keepdim=True) + EPS) * (1 + sc) + sh

    n = ln(x, mo[:D], mo[D:2 * D])
    q, k, v = n @ bf(w["sa_q"]).T, n @ bf(w["sa_k"]).T, n @ bf(w["sa_v"]).T
    a = torch.empty(B * T, D, dtype=torch.float64)
    for b in range(B):
        r_ = slice(b * T, (b + 1) * T)
        a[r_] = _attn(_rope(_rms(q[r_], bf(w["sa_qn"]), H, EPS), d(rc), d(rs), H),
                      _rope(_rms(k[r_], bf(w["sa_kn"]), H, EPS), d(rc), d(rs), H), v[r_], H)
    x = x + mo[2 * D:] * (a @ bf(w["sa_o"]).T)
    n = ln(x, mc[:D], mc[D:2 * D])
    qc = _rms(n @ bf(w["ca_q"]).T, bf(w["ca_qn"]), H, EPS)
    kv = [_ctx_kv(w, c) for c in ctxs]
    for b in range(B):
        r_ = slice(b * T, (b + 1) * T)
        a[r_] = _attn(qc[r_], kv[b][0], kv[b][1], H, L - REALS[b])
    an = _attn(qc[:T], kv[2][0], kv[2][1], H, L - REALS[2])
    a[:T] = torch.from_numpy(oracle.nag(a[:T].numpy(), an.numpy(), *NAG)).double()
    x = x + mc[2 * D:] * (a @ bf(w["ca_o"]).T)
    n = ln(x, mm[:D], mm[D:2 * D])
    h = n @ bf(w["mlp1"]).T
    h = 0.5 * h * (1 + torch.erf(h / np.sqrt(2)))
    x = x + mm[2 * D:] * (h @ bf(w["mlp2"]).T)
    err = (X.cpu().double() - x).abs()
    assert err.max().item() <= 1e-3 and err.mean().item() <= 5e-5, (err.max().item(), err.mean().item())


def test_dit_sample_in_cpp_matches_the_python_driven_loop(gpu):
    """kiln_dit_sample (sample() with the DiT as its model, the whole loop in C++: pipeline.cu:415-598) against
    the same sampler driving Dit.forward from Python: CFG of the pair in one batched forward with NAG on the
    prompt is bit-identical; the unbatched CFG path (prompt pass with NAG, negative pass without) agrees to
    fp16-path noise; NAG switched off below nag_sigma_end changes the result."""
    from kiln_amd import sampler
    g = torch.Generator().manual_seed(38)
    d, _, _ = _make_dit(g, 2)
    cc = [d.cache_context(torch.randn(r, DCTX, generator=g).to(DEV), length=L) for r in REALS]
    nag = dit.Nag(cc[2], *NAG)
    shape = (16, 2 * Hp, 2 * Wp)
    noise = torch.randn(*shape, generator=g).to(DEV)
    kw = dict(steps=4, shift=3.0, cfg=3.0, cfg_until=0.5, seed=7, noise=noise)

    def model(outs, x, t, cfg_now):
        if cfg_now:
            d.forward(outs, x, t, cc[:2], nag=nag)
        else:
            d.forward(outs[:1], x, t, cc[:1], nag=nag)

    ref = torch.empty(*shape, device=DEV)
    sampler.sample_euler(model, ref, noise, sampler.flow_sigmas(4, 3.0), cfg=3.0, cfg_until=0.5)
    x = torch.empty_like(ref)
    d.sample(x, cc[0], neg=cc[1], nag=nag, **kw)
    torch.cuda.synchronize()
    assert torch.isfinite(x).all() and torch.equal(x, ref)
    xu = torch.empty_like(ref)
    d.sample(xu, cc[0], neg=cc[1], nag=nag, batch_cfg=False, **kw)
    torch.cuda.synchronize()
    assert (xu - ref).abs().max().item() <= 2e-2
    xo = torch.empty_like(ref)
    d.sample(xo, cc[0], neg=cc[1], nag=nag, nag_sigma_end=2.0, **kw)  # every sigma < 2: NAG never applies
    xn = torch.empty_like(ref)
    d.sample(xn, cc[0], neg=cc[1], **kw)
    torch.cuda.synchronize()
    assert torch.equal(xo, xn) and not torch.equal(xo, x)


def test_profiler_categories_of_a_forward(gpu):
    """kiln_prof_* (the reference's ProfScope / prof_report, engine/src/kernels.cu:14-58): a profiled forward of
    the CFG pair reports the attention, GEMM, LayerNorm, matvec and elementwise categories; nested entry points
    are counted once (the category sum stays within the forward's own event-timed duration); a disabled profiler
    records nothing."""
    g = torch.Generator().manual_seed(39)
    d, _, _ = _make_dit(g, 2)
    cc = [d.cache_context(torch.randn(r, DCTX, generator=g).to(DEV), length=L) for r in REALS]
    lat = torch.randn(16, 2 * Hp, 2 * Wp, generator=g).to(DEV)
    outs = [torch.empty_like(lat) for _ in range(B)]
    d.forward(outs, lat, 0.5, cc[:B], nag=dit.Nag(cc[2], *NAG))  # warm
    kiln_amd.prof_enable(True)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    d.forward(outs, lat, 0.5, cc[:B], nag=dit.Nag(cc[2], *NAG))
    e1.record()
    cats, text = kiln_amd.prof_report()
    kiln_amd.prof_enable(False)
    torch.cuda.synchronize()
    print(text)
    for c in ("attention", "gemm_tc16", "layernorm", "matvec", "gemm_fp32", "eltwise"):
        assert c in cats and cats[c][1] > 0 and cats[c][0] > 0, (c, cats)
    # 2 blocks: per block one self-attention and one cross-attention section, 3 LN16, 4 linear16 (O, O, MLP x 2) and
    # the two projections inside the fused sections
    assert cats["attention"][1] == 4 and cats["layernorm"][1] == 2 * 3 + 1 and cats["gemm_tc16"][1] == 2 * 6
    total = sum(v[0] for v in cats.values())
    assert total <= e0.elapsed_time(e1) * 1.05 + 0.05
    kiln_amd.prof_enable(True)
    kiln_amd.prof_enable(False)
    cats, _ = kiln_amd.prof_report()
    assert cats == {}
