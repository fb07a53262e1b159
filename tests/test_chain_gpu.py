"""Context chains of the cross-attention launch: one unit per (query tile, head) runs every context's keys in turn
(item 0's positive and NAG-negative contexts back to back on the same Q registers, then item 1's), instead of one
unit per (context, query tile, head). Each context's softmax runs the same key loop in the same order either way,
so the outputs are bit-identical to the per-context units; the chained call is also held to the oracle.
Chains are the default for launches whose per-context units take more than one round of the resident slots;
KILN_CHAIN=0 selects the per-context units for the comparison."""
import os

import numpy as np
import pytest
import torch

import kiln_amd
import oracle
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
H, D = 16, 128


def _run(env, fn):
    old = {"KILN_CHAIN": os.environ.get("KILN_CHAIN")}
    os.environ.pop("KILN_CHAIN", None)
    os.environ.update(env)
    try:
        out = fn()
        torch.cuda.synchronize()
        return out
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


# every shape takes more than one round of per-context units (the launches that chain): config 5's, ragged query
# and key counts, npad, one item with its NAG negative (a two-context chain on one Q tile), no NAG
@pytest.mark.parametrize("T,Ls,neg,B,out32", [(3456, (512, 512), (512, 0), 2, False), (3000, (300, 77), (26, 486), 2, False),
                                              (2600, (97, 512), None, 2, True), (4100, (512,), (40, 472), 1, True)])
def test_context_chain_matches_per_context_units(gpu, T, Ls, neg, B, out32):
    print(f"[case] chain T={T} Ls={Ls} neg={neg} B={B} out32={out32}", flush=True)
    g = torch.Generator().manual_seed(T + B)
    q = torch.randn(B * T, H * D, generator=g).half()
    qw = (1 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16)
    ctx = [(torch.randn(L, H * D, generator=g).half(), torch.randn(L, H * D, generator=g).half()) for L in Ls]
    nctx = None if neg is None else (torch.randn(neg[0], H * D, generator=g).half(),
                                     torch.randn(neg[0], H * D, generator=g).half())
    kvps = [kiln_amd.kv_prepare(k.to(DEV), v.to(DEV), H) for k, v in ctx]
    kvn = None if nctx is None else kiln_amd.kv_prepare(nctx[0].to(DEV), nctx[1].to(DEV), H)
    qd, wd = q.to(DEV), qw.to(DEV)
    odt = torch.float32 if out32 else torch.float16

    def call():
        o = torch.full((B * T, H * D), float("nan"), dtype=odt, device=DEV)
        on = torch.full((T, H * D), float("nan"), dtype=odt, device=DEV)
        kw = {} if kvn is None else dict(kvp_neg=kvn, Lk_neg=neg[0], npad_neg=neg[1], out_neg=on)
        kiln_amd.cross_attn_nag(o, qd, B, T, H, kvps, list(Ls), [0] * B, q_norm_w=wd, **kw)
        return o, on
    ref, ref_n = _run({"KILN_CHAIN": "0"}, call)
    got, got_n = _run({}, call)  # the default: context chains
    assert torch.equal(got, ref), "the context chain differs from per-context units"
    if kvn is not None:
        assert torch.equal(got_n, ref_n), "the context chain's NAG negative output differs"
    # and against the oracle on sampled rows
    rows = np.sort(np.random.default_rng(T).choice(T, size=min(T, 96), replace=False))
    wb = qw.view(torch.int16).numpy().view(np.uint16)
    o = got.float().cpu().numpy()
    for b in range(B):
        qn = oracle.rmsnorm_rows(q[b * T:(b + 1) * T][rows].float().numpy(), wb).reshape(len(rows), H * D)
        z = oracle.attn_f64(qn, ctx[b][0].float().numpy(), ctx[b][1].float().numpy(), H)
        if b == 0 and nctx is not None:
            z = oracle.nag(z, oracle.attn_f64(qn, nctx[0].float().numpy(), nctx[1].float().numpy(), H, npad=neg[1]))
        bar = dict(max_abs=6e-3, mean_abs=6e-4) if (b == 0 and nctx is not None) else {}
        assert_close(o[b * T:(b + 1) * T][rows], z, f"chain cross T={T} item {b}", **bar)
