"""Parity of configs 3 and 5's cross-attention + NAG on the inputs those configs name.

Config 3: 1536 image-token queries (16 heads x 128, Q from N(0,1) activations projected by a random-init
W_q, QK-RMSNorm) over a positive and a negative context of 512 Qwen3-0.6B-sized tokens: [512, 1024] N(0,1)
embeddings projected to 2048 by the block's random-init W_k / W_v through Dit::cache_context
(kiln_dit_cache_context, engine/src/dit.cu:217-234), then the NAG combine (s = 5, tau = 2.5, alpha = 0.25,
engine/src/dit.cu:295-324).

Config 5: the x16 cross-attention section at T = 48 x 72 = 3456 for the CFG pair (cross-Q projection with the Q
RMSNorm in its epilogue, each item against its cached context, the NAG negative of item 0, the combine),
engine/src/dit.cu:473-488, on sampled query rows.

Both against the double-accumulation oracle (oracle.attn_f64 + oracle.nag, K/V and Q projected in float64 from
the same fp16 / bf16 values) at the BASELINE bar (max-abs 2e-3, mean-abs 2e-4), fp16 and fp32 outputs.
"""
import numpy as np
import pytest
import torch

import kiln_amd
import oracle
from kiln_amd import dit
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
H, HD, CTX = 16, 128, 1024
D = H * HD
NAG = (5.0, 2.5, 0.25)


def _linear_init(g, o, i):
    """torch.nn.Linear's default weight init U(+-1/sqrt(in)), as bf16 (a checkpoint's dtype)."""
    return ((torch.rand(o, i, generator=g) * 2 - 1) / i ** 0.5).to(torch.bfloat16)


def _one_block_dit(g):
    """A one-block Dit of the 2B shapes (16 heads, D = 2048, 1024-d contexts) with random-init weights and norm
    weights 1 (torch's RMSNorm init); returns it and the host weights."""
    d = dit.Dit(1, H, ctx_dim=CTX)
    ones = torch.ones(HD, dtype=torch.bfloat16)
    w = dict(sa_q=_linear_init(g, D, D), sa_k=_linear_init(g, D, D), sa_v=_linear_init(g, D, D),
             sa_o=_linear_init(g, D, D), ca_q=_linear_init(g, D, D), ca_o=_linear_init(g, D, D),
             ca_k=_linear_init(g, D, CTX), ca_v=_linear_init(g, D, CTX), mlp1=_linear_init(g, 4 * D, D),
             mlp2=_linear_init(g, D, 4 * D), sa_qn=ones, sa_kn=ones, ca_qn=ones, ca_kn=ones,
             mod=[_linear_init(g, 256, D), _linear_init(g, 3 * D, 256)] * 3)
    d.set_block(0, **{k: (v.to(DEV) if torch.is_tensor(v) else [m.to(DEV) for m in v]) for k, v in w.items()})
    return d, w


def _ctx_ref(w, ctx):
    """K = rmsnorm(ctx W_k^T; ca_kn), V = ctx W_v^T in float64 from the bf16 weights (Dit::cache_context)."""
    c = ctx.double()
    k = (c @ w["ca_k"].double().T).numpy()
    kn = oracle.rmsnorm_rows(k, w["ca_kn"].view(torch.int16).numpy().view(np.uint16)).reshape(k.shape)
    return kn, (c @ w["ca_v"].double().T).numpy()


@pytest.mark.parametrize("out32", [False, True])
def test_config3_cross_attention_nag_own_inputs(gpu, out32):
    T, L = 1536, 512
    print(f"[case] config 3 own inputs out32={out32}", flush=True)
    g = torch.Generator().manual_seed(303)
    d, w = _one_block_dit(g)
    ctx_pos, ctx_neg = torch.randn(L, CTX, generator=g), torch.randn(L, CTX, generator=g)
    cp, cn = d.cache_context(ctx_pos.to(DEV)), d.cache_context(ctx_neg.to(DEV))
    X = torch.randn(T, D, generator=g)
    q = (X.double() @ _linear_init(g, D, D).double().T).float().half()  # projected queries, fp16
    odt = torch.float32 if out32 else torch.float16
    out = torch.empty(T, D, dtype=odt, device=DEV)
    on = torch.empty(T, D, dtype=odt, device=DEV)
    kiln_amd.cross_attn_nag(out, q.to(DEV), 1, T, H, [cp.kv(0)], [L], [0], q_norm_w=w["ca_qn"].to(DEV),
                            kvp_neg=cn.kv(0), Lk_neg=L, npad_neg=0, out_neg=on, scale=NAG[0], tau=NAG[1],
                            alpha=NAG[2])
    torch.cuda.synchronize()
    qn = oracle.rmsnorm_rows(q.float().numpy(), w["ca_qn"].view(torch.int16).numpy().view(np.uint16)).reshape(T, D)
    zp = oracle.attn_f64(qn, *_ctx_ref(w, ctx_pos), H)
    zn = oracle.attn_f64(qn, *_ctx_ref(w, ctx_neg), H)
    assert_close(on.float().cpu().numpy(), zn, f"config 3 NAG negative attention out32={out32}")
    assert_close(out.float().cpu().numpy(), oracle.nag(zp, zn, *NAG), f"config 3 NAG combine out32={out32}")


@pytest.mark.parametrize("out32", [False, True])
def test_config5_cross_attention_nag_x16(gpu, out32):
    Hp, Wp, B, L = 48, 72, 2, 512
    T = Hp * Wp
    print(f"[case] config 5 x16 cross-attention + NAG T={T} out32={out32}", flush=True)
    g = torch.Generator().manual_seed(505)
    d, w = _one_block_dit(g)
    ctxs = [torch.randn(L, CTX, generator=g) for _ in range(3)]  # prompt, unconditional, NAG negative
    cc = [d.cache_context(c.to(DEV)) for c in ctxs]
    x16 = torch.randn(B * T, D, generator=g).half()  # the block's modulated LayerNorm output, fp16
    wq = w["ca_q"].half()  # weight_to_f16 of the block's cross-Q weight
    wp = kiln_amd.linear16_prepare_weight(wq.to(DEV))
    odt = torch.float32 if out32 else torch.float16
    out = torch.empty(B * T, D, dtype=odt, device=DEV)
    on = torch.empty(T, D, dtype=odt, device=DEV)
    kiln_amd.dit_cross_attn_x16(out, x16.to(DEV), wp, B, T, H, [cc[0].kv(0), cc[1].kv(0)], [L, L], [0, 0],
                                w["ca_qn"].to(DEV), kvp_neg=cc[2].kv(0), Lk_neg=L, npad_neg=0, out_neg=on,
                                scale=NAG[0], tau=NAG[1], alpha=NAG[2])
    torch.cuda.synchronize()
    o = out.float().cpu().numpy()
    rows = np.sort(np.random.default_rng(5).choice(T, size=96, replace=False))
    kv = [_ctx_ref(w, c) for c in ctxs]
    wqn = w["ca_qn"].view(torch.int16).numpy().view(np.uint16)
    for b in range(B):
        qb = (x16[b * T:(b + 1) * T][rows].double() @ wq.double().T).numpy()
        qn = oracle.rmsnorm_rows(qb, wqn).reshape(len(rows), D)
        z = oracle.attn_f64(qn, *kv[b], H)
        if b == 0:
            z = oracle.nag(z, oracle.attn_f64(qn, *kv[2], H), *NAG)
        assert_close(o[b * T:(b + 1) * T][rows], z, f"config 5 cross + NAG item {b} out32={out32}")
