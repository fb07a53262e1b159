"""The Cosmos-Predict2 DiT forward composed from the library's entry points.

block_forward16 mirrors the block loop of the reference's Dit::forward_batch for G.fp16 && G.tc16
(engine/src/dit.cu:455-494); forward16 adds the step tables, patch embedding, final layer and the first-block
step cache (dit.cu:357-546); block_forward32 is the fp32 branch of the block (dit.cu:495-530). The fp16 block:

    N16 = layernorm_mod16(X; shift, scale of the self-attention modulation)
    Q, K, V = linear16(N16, sa_q / sa_k / sa_v)   one launch on [Wq; Wk; Wv] whose epilogue applies
    A16 = attention16(rmsnorm+rope(Q), ...)       QK-RMSNorm + RoPE and writes fp16 Q / prepared K/V,
                                                  then one attention launch (kiln_dit_self_attn_x16)
    X += gate * linear16(A16, sa_o)                                      RESID epilogue
    N16 = layernorm_mod16(X; cross-attention modulation)
    Q = linear16(N16, ca_q)                       epilogue applies the Q RMSNorm, fp16 Q; then the
    A16 = attention16(rmsnorm(Q), ctx K/V) + NAG  attention of all contexts + NAG (kiln_dit_cross_attn_x16)
    X += gate * linear16(A16, ca_o)
    N16 = layernorm_mod16(X; MLP modulation)
    H16 = GELU(linear16(N16, mlp1))                                      GELU16 epilogue
    X += gate * linear16(H16, mlp2)

The modulation vector of a block is [9 * D] fp32: (shift, scale, gate) for self-attention, cross-attention
and the MLP (engine/src/dit.cu:266-268, used at :460-493). Context K/V are prepared once per generation and
block (Dit::cache_context, engine/src/dit.cu:217-234): K = rmsnorm(ctx @ ca_k^T; ca_kn), V = ctx @ ca_v^T.
Every call below goes to the HIP library; there is no CPU path.
"""
import numpy as np
import torch

from . import (KILN_EPI_GELU16, KILN_EPI_RESID, add_gated, dit_cross_attn_x16, dit_self_attn_x16,
               kv_prepare, layernorm_mod, lib, linear16, linear16_prepare_weight, linear_f32, matvec, matvec_grouped,
               patchify, rel_l1, rmsnorm, silu, sub, unpatchify, attention_exact, gelu, rope_half, nag_combine)

HD = 128


class Block16:
    """The weights of one DiT block in the layout the fp16 path consumes: every linear16 weight prepared at
    load (kiln_linear16_prepare_weight; Q/K/V stacked into one [3D, D] weight), norm weights bf16 [128]."""

    def __init__(self, sa_qkv, sa_o, ca_q, ca_o, mlp1, mlp2, sa_qn, sa_kn, ca_qn, ca_kn, ca_k=None, ca_v=None,
                 mod=None):
        self.sa_qkv = linear16_prepare_weight(sa_qkv)
        self.sa_o = linear16_prepare_weight(sa_o)
        self.ca_q = linear16_prepare_weight(ca_q)
        self.ca_o = linear16_prepare_weight(ca_o)
        self.mlp1 = linear16_prepare_weight(mlp1)
        self.mlp2 = linear16_prepare_weight(mlp2)
        self.sa_qn, self.sa_kn, self.ca_qn, self.ca_kn = sa_qn, sa_kn, ca_qn, ca_kn
        self.ca_k, self.ca_v = ca_k, ca_v  # fp32 [D, Dctx] context projections (used by prepare_context)
        # adaLN modulation weights, bf16: (sa1 [256, D], sa2 [3D, 256], ca1, ca2, mlp1, mlp2), dit.cu:266-268
        self.mod = mod
        self.D = sa_o.shape[0]
        self.F = mlp1.shape[0]

    def prepare_context(self, ctx, eps=1e-6):
        """Dit::cache_context for this block (engine/src/dit.cu:217-234): the real rows of a context
        [L, Dctx] fp32 -> prepared K/V (K RMS-normed with ca_kn)."""
        k = ctx @ self.ca_k.t()
        v = ctx @ self.ca_v.t()
        return kv_prepare(k, v, self.D // HD, k_norm_w=self.ca_kn, eps=eps)


class Workspace:
    """Activation buffers of one forward at B items x T tokens (the reference's arena slices N, big, A)."""

    def __init__(self, B, T, D, F, device):
        R = B * T
        self.n16 = torch.empty(R, D, dtype=torch.float16, device=device)
        self.q16 = torch.empty(R * D * 2, dtype=torch.uint8, device=device)  # fp16 cross-attention Q
        self.a16 = torch.empty(R, D, dtype=torch.float16, device=device)
        self.an16 = torch.empty(T, D, dtype=torch.float16, device=device)
        self.h16 = torch.empty(R, F, dtype=torch.float16, device=device)
        self.attn_ws = torch.empty(lib().kiln_dit_self_attn_x16_workspace_bytes(B, T, D // HD), dtype=torch.uint8,
                                   device=device)


def block_forward16(X, mods, blk, ws, B, T, rope, ctx, nag=None, eps=1e-6):
    """X [B*T, D] fp32 (updated in place) through one block. mods [9*D] fp32; rope = (cos, sin) [T, 64];
    ctx: per item (prepared K/V, real rows, padding rows); nag: None or (prepared K/V, real, padding, scale,
    tau, alpha) for item 0."""
    D, H = blk.D, blk.D // HD
    mo, mc, mm = mods[0:3 * D], mods[3 * D:6 * D], mods[6 * D:9 * D]
    # self-attention: the Q/K/V projection's epilogue applies the QK-RMSNorm and RoPE and writes fp16 Q and the
    # prepared K/V, then the attention of the B items (kiln_dit_self_attn_x16)
    layernorm_mod(ws.n16, X, mo[D:2 * D], mo[0:D], eps)
    dit_self_attn_x16(ws.a16, ws.n16, blk.sa_qkv, B, T, H, blk.sa_qn, blk.sa_kn, rope, eps=eps, workspace=ws.attn_ws)
    linear16(X, ws.a16, blk.sa_o, epi=KILN_EPI_RESID, gate=mo[2 * D:3 * D])
    # cross-attention, each item against its own context (+ NAG on item 0): the cross-Q projection's epilogue
    # applies the Q RMSNorm and writes fp16 Q (kiln_dit_cross_attn_x16)
    layernorm_mod(ws.n16, X, mc[D:2 * D], mc[0:D], eps)
    args = dict(q_norm_w=blk.ca_qn, eps=eps, workspace=ws.q16)
    if nag is not None:
        args.update(kvp_neg=nag[0], Lk_neg=nag[1], npad_neg=nag[2], out_neg=ws.an16, scale=nag[3], tau=nag[4],
                    alpha=nag[5])
    dit_cross_attn_x16(ws.a16, ws.n16, blk.ca_q, B, T, H, [c[0] for c in ctx[:B]], [c[1] for c in ctx[:B]],
                       [c[2] for c in ctx[:B]], **args)
    linear16(X, ws.a16, blk.ca_o, epi=KILN_EPI_RESID, gate=mc[2 * D:3 * D])
    # MLP
    layernorm_mod(ws.n16, X, mm[D:2 * D], mm[0:D], eps)
    linear16(ws.h16, ws.n16, blk.mlp1, epi=KILN_EPI_GELU16)
    linear16(X, ws.h16, blk.mlp2, epi=KILN_EPI_RESID, gate=mm[2 * D:3 * D])
    return X


class Block32:
    """One block's weights for the fp32 branch (G.fp16 off, the engine's --fp32): bf16 [out, in] linear weights
    read as fp32 (the reference's weight_f32), norm weights bf16 [128]."""

    def __init__(self, sa_q, sa_k, sa_v, sa_o, ca_q, ca_o, mlp1, mlp2, sa_qn, sa_kn, ca_qn):
        self.sa_q, self.sa_k, self.sa_v, self.sa_o = sa_q, sa_k, sa_v, sa_o
        self.ca_q, self.ca_o, self.mlp1, self.mlp2 = ca_q, ca_o, mlp1, mlp2
        self.sa_qn, self.sa_kn, self.ca_qn = sa_qn, sa_kn, ca_qn
        self.D, self.F = sa_o.shape[0], mlp1.shape[0]


def block_forward32(X, mods, blk, B, T, rope, ctx, nag=None, eps=1e-6):
    """The fp32 branch of the block loop (engine/src/dit.cu:495-530): fp32 activations throughout, fp32 linear
    layers (kiln_linear_f32), per-head RMSNorm + rope_half on Q/K, the exact fp32 attention per item
    (kiln_attn_fwd_exact: attention() with G.fp16 off, kernels.cu:840-865), add_gated residuals, fp32 GELU. ctx: per item (K fp32 [L, D], V fp32 [L, D], padding
    rows) with K already RMS-normed (Dit::cache_context); nag: None or (K, V, padding, scale, tau, alpha)."""
    D, H = blk.D, blk.D // HD
    R = B * T
    dev = X.device
    mo, mc, mm = mods[0:3 * D], mods[3 * D:6 * D], mods[6 * D:9 * D]
    N = torch.empty(R, D, device=dev)
    Q, K, V, A, Y = (torch.empty(R, D, device=dev) for _ in range(5))
    rc, rs = rope
    layernorm_mod(N, X, mo[D:2 * D], mo[0:D], eps)
    linear_f32(Q, N, blk.sa_q)
    linear_f32(K, N, blk.sa_k)
    linear_f32(V, N, blk.sa_v)
    rmsnorm(Q, Q, blk.sa_qn, rows=R * H, dim=HD, eps=eps)
    rmsnorm(K, K, blk.sa_kn, rows=R * H, dim=HD, eps=eps)
    for b in range(B):
        rows = slice(b * T, (b + 1) * T)
        rope_half(Q[rows], T, H, HD, rc, rs)
        rope_half(K[rows], T, H, HD, rc, rs)
        attention_exact(A[rows], Q[rows], K[rows], V[rows], T, T, H, HD)
    linear_f32(Y, A, blk.sa_o)
    add_gated(X, Y, mo[2 * D:3 * D])
    layernorm_mod(N, X, mc[D:2 * D], mc[0:D], eps)
    linear_f32(Q, N, blk.ca_q)
    rmsnorm(Q, Q, blk.ca_qn, rows=R * H, dim=HD, eps=eps)
    for b in range(B):
        rows = slice(b * T, (b + 1) * T)
        attention_exact(A[rows], Q[rows], ctx[b][0], ctx[b][1], T, ctx[b][0].shape[0], H, HD, npad=ctx[b][2])
    if nag is not None:
        An = torch.empty(T, D, device=dev)
        attention_exact(An, Q[0:T], nag[0], nag[1], T, nag[0].shape[0], H, HD, npad=nag[2])
        nag_combine(A[0:T], An, nag[3], nag[4], nag[5])
    linear_f32(Y, A, blk.ca_o)
    add_gated(X, Y, mc[2 * D:3 * D])
    layernorm_mod(N, X, mm[D:2 * D], mm[0:D], eps)
    Hid = torch.empty(R, blk.F, device=dev)
    linear_f32(Hid, N, blk.mlp1)
    gelu(Hid)
    linear_f32(Y, Hid, blk.mlp2)
    add_gated(X, Y, mm[2 * D:3 * D])
    return X


class StepWeights:
    """The DiT's per-step weights outside the blocks, bf16 (engine/src/dit.cu:53-59, 242-272): the timestep MLP
    t_lin1 [D, D], t_lin2 [3D, D] (the adaLN-LoRA vector), t_norm [D]; the final layer's modulation
    final_mod1 [256, D], final_mod2 [2D, 256]; the patch embedder x_embed [D, 68] and final_lin [64, D]."""

    def __init__(self, t_lin1, t_lin2, t_norm, final_mod1, final_mod2, x_embed, final_lin):
        self.t_lin1, self.t_lin2, self.t_norm = t_lin1, t_lin2, t_norm
        self.final_mod1, self.final_mod2 = final_mod1, final_mod2
        self.x_embed, self.final_lin = x_embed, final_lin
        self._mod1 = None  # the blocks' modulation weights stacked for step_tables (built on first use)


def timestep_sinusoid(t, D):
    """The host-side sinusoid of Dit::step_tables (engine/src/dit.cu:246-251), fp32 arithmetic: cos(t e_i) and
    sin(t e_i), e_i = exp(-i ln(10000) / (D/2))."""
    i = np.arange(D // 2, dtype=np.float32)
    e = np.exp(i * np.float32(-np.log(np.float32(10000.0))) / np.float32(D // 2)).astype(np.float32)
    te = (np.float32(t) * e).astype(np.float32)
    return np.concatenate([np.cos(te), np.sin(te)]).astype(np.float32)


def step_tables(t, sw, blocks, device, eps=1e-6):
    """Dit::step_tables (engine/src/dit.cu:242-272): the modulation vectors of every block ([9D] each) and of
    the final layer ([2D]), from the timestep t. Returns (mods [nblocks, 9D], fmod [2D])."""
    D = sw.t_lin1.shape[0]
    s = torch.from_numpy(timestep_sinusoid(t, D)).to(device)
    s1 = torch.empty(D, device=device)
    lora = torch.empty(3 * D, device=device)
    temb = torch.empty(D, device=device)
    h = torch.empty(256, device=device)
    matvec(s1, sw.t_lin1, s)
    silu(s1, s1)
    matvec(lora, sw.t_lin2, s1)
    rmsnorm(temb, s, sw.t_norm, rows=1, dim=D, eps=eps)
    silu(temb, temb)  # every modulation MLP starts with SiLU
    # every block's three modulation MLPs in two launches: [nblocks*3*256, D] first layers on temb, then the
    # second layers [nblocks*3, 3D, 256] each on its own hidden vector, + lora
    if getattr(sw, "_mod1", None) is None or sw._mod_blocks != [id(b) for b in blocks]:
        sw._mod1 = torch.cat([blk.mod[2 * j] for blk in blocks for j in range(3)]).contiguous()
        sw._mod2 = torch.stack([blk.mod[2 * j + 1] for blk in blocks for j in range(3)]).contiguous()
        sw._mod_blocks = [id(b) for b in blocks]
    hid = torch.empty(len(blocks) * 3, 256, device=device)
    matvec(hid.view(-1), sw._mod1, temb)
    mods = torch.empty(len(blocks), 9 * D, device=device)
    matvec_grouped(mods.view(len(blocks) * 3, 3 * D), sw._mod2, hid, add=lora)
    fmod = torch.empty(2 * D, device=device)
    matvec(h, sw.final_mod1, temb)
    matvec(fmod, sw.final_mod2, h, add=lora[:2 * D])
    return mods, fmod


class StepCache:
    """The first-block step cache (Dit::StepCache, engine/src/models.h:66-76): across the steps of one sampling
    run, when block 0's residual moved less than `threshold` (relative L1) since the last full forward, the
    forward reuses that forward's residual of blocks 1..N-1 instead of running them. `allow` is set per step by
    the sampler."""

    def __init__(self, threshold):
        self.threshold, self.allow, self.valid, self.skipped = threshold, False, False, False
        self.R, self.r0, self.resid, self.last_change = 0, None, None, 0.0
        self.acc = None


def forward16(outs, latent, t, sw, blocks, ws, B, rope, ctx, nag=None, eps=1e-6, sc=None):
    """Dit::forward_batch on the fp16 path (engine/src/dit.cu:357-546, step cache at :404-433, :532-536): every batch
    item starts from the same latent [16, Hl, Wl]; outs: B latents [16, Hl, Wl] (the velocity predictions).
    ctx[b] = (prepared K/V of block i -> list over blocks, real rows, padding rows); nag as in block_forward16
    but with per-block prepared K/V lists."""
    Hl, Wl = latent.shape[1], latent.shape[2]
    T = (Hl // 2) * (Wl // 2)
    D = sw.t_lin1.shape[0]
    dev = latent.device
    mods, fmod = step_tables(t, sw, blocks, dev, eps)
    tok = torch.empty(T, 68, device=dev)
    patchify(tok, latent)
    X = torch.empty(B * T, D, device=dev)
    linear_f32(X[:T], tok, sw.x_embed)
    for b in range(1, B):
        X[b * T:(b + 1) * T].copy_(X[:T])
    use_cache = sc is not None and sc.threshold > 0
    if use_cache:
        R = B * T
        if sc.R != R or sc.r0 is None:
            sc.valid, sc.R = False, R
            sc.r0 = torch.empty(R, D, device=dev)
            sc.resid = torch.empty(R, D, device=dev)
            sc.acc = torch.empty(2, device=dev)
        X0 = X.clone()  # input of block 0
        sc.skipped = False
    for i, blk in enumerate(blocks):
        if use_cache and i == 1:
            sub(X0, X, X0)  # block 0's residual of this step
            if sc.valid:
                rel_l1(X0, sc.r0, sc.acc)
                h = sc.acc.cpu()  # synchronizes, as the reference's cudaMemcpy does
                sc.last_change = float(h[0] / h[1]) if h[1] > 0 else 1.0
                if sc.allow and sc.last_change < sc.threshold:
                    add_gated(X, sc.resid)  # X = block-0 output + cached residual of blocks 1..N-1
                    sc.skipped = True
                    break
            sc.r0.copy_(X0)
            sc.resid.copy_(X)  # block-0 output, turned into the residual below
        cb = [(c[0][i], c[1], c[2]) for c in ctx]
        nb = None if nag is None else (nag[0][i],) + tuple(nag[1:])
        block_forward16(X, mods[i], blk, ws, B, T, rope, cb, nag=nb, eps=eps)
    if use_cache and not sc.skipped:
        sub(sc.resid, X, sc.resid)  # the residual of blocks 1..N-1
        sc.valid = True
    N = torch.empty_like(X)
    layernorm_mod(N, X, fmod[D:2 * D], fmod[:D], eps)
    y = torch.empty(B * T, 64, device=dev)
    linear_f32(y, N, sw.final_lin)
    for b in range(B):
        unpatchify(outs[b], y[b * T:(b + 1) * T])
    return outs
