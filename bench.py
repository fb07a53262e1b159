#!/usr/bin/env python3
"""Benchmark of the MI355X fused attention path (one JSON line on stdout).

Headline (`value`): DiT self-attention at 1024x1024 (T = 64x64 = 4096 tokens), CFG batch B=2, H=16, d=128,
fp16 Q/K/V from random-init linear projections of N(0,1) activations, QK-RMSNorm + Cosmos 3D RoPE fused
One "step" = one call of the fused path (K/V prepare pass + attention kernel) with
inputs resident in HBM. FLOP = 4*B*H*Tq*Tk*d (the reference's formula, bench/flash_test.cu:62).

The same line also carries: the S=1536 CFG pair (config 2), the attention ms of a full 28-block DiT step
at 768x1152 (config 5: self + cross + NAG), the roofline of the dominant kernel (k_attn_fwd, timed with HIP
events around its launches inside the call's prepare -> attention sequence, on its stream) and the CPU baseline (the reference's fp32 two-pass attention restated in
C, oracle/oracle.c, on a bounded sample of config 4, on this host's cores).

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "attention TFLOP/s + % fp16 MFMA peak at S=1536/4096; ms attn per DiT step"
PEAK_TFLOPS = 2516.6  # MI355X dense fp16 MFMA: 256 CU x 2.4 GHz x 4096 flop/clk
H, D = 16, 128
WARM_S = 0.2  # seconds of untimed sustained work before each timed loop


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_dit_inputs(torch, B, T, seed, dev):
    """Q/K/V = X W^T (fp16) with X ~ N(0,1) [B*T, 2048], W ~ U(+-1/sqrt(2048)) (torch Linear init)."""
    g = torch.Generator(device=dev).manual_seed(seed)
    X = torch.randn(B * T, H * D, generator=g, device=dev)
    outs = []
    for _ in range(3):
        W = (torch.rand(H * D, H * D, generator=g, device=dev) * 2 - 1) / (H * D) ** 0.5
        outs.append((X @ W.T).half())
    del X
    return outs


class Timer:
    """HIP events on the current stream (the stream every kiln call is enqueued on)."""

    def __init__(self, torch):
        self.torch = torch

    def run_inner(self, before, fn, steps, warmup):
        """Mean duration of fn() when each call follows before() (events around fn only): the attention kernel
        inside the call's prepare -> attention sequence, i.e. at the clock the chip runs it at in the timed call
        (back to back, with no prepare pass between, the same launches run at the power limit's lower clock)."""
        torch = self.torch
        for _ in range(warmup):
            before()
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < WARM_S:
            for _ in range(max(1, warmup)):
                before()
                fn()
            torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        for a, b in ev:
            before()
            a.record()
            fn()
            b.record()
        torch.cuda.synchronize()
        return sum(a.elapsed_time(b) for a, b in ev) / steps

    def run(self, fn, steps, warmup):
        torch = self.torch
        # untimed warm-up: `warmup` calls, then more until ~WARM_S of GPU work has run, so the timed loop
        # sees the clock the GPU settles at under sustained matrix-core load (it ramps and overshoots
        # for several ms after an idle period)
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < WARM_S:
            for _ in range(max(1, warmup)):
                fn()
            torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps


def self_attn_case(torch, kiln_amd, Hp, Wp, B, seed, dev):
    T = Hp * Wp
    q, k, v = make_dit_inputs(torch, B, T, seed, dev)
    qw = torch.ones(D, dtype=torch.bfloat16, device=dev)  # torch RMSNorm init
    kw = torch.ones(D, dtype=torch.bfloat16, device=dev)
    c, s = kiln_amd.cosmos_rope_tables(Hp, Wp)
    rope = (c.to(dev), s.to(dev))
    out = torch.empty_like(q)
    ws = torch.empty(kiln_amd.dit_self_attn_workspace_bytes(B, T, H), dtype=torch.uint8, device=dev)

    def step():
        kiln_amd.dit_self_attn(out, q, k, v, B, T, H, qw, kw, rope, workspace=ws)

    # the same work split into its two passes, so the attention kernel can be timed alone
    kvps = [kiln_amd.kv_prepare(k[b * T:(b + 1) * T], v[b * T:(b + 1) * T], H, k_norm_w=kw, rope=rope)
            for b in range(B)]

    def main_kernel():
        kiln_amd.attn_prepped_batch(out, q, kvps, T, T, H, q_norm_w=qw, rope=rope)

    def prep_only():  # the call's first pass into the same buffers (kiln_kv_prepare, no allocation)
        L = kiln_amd.lib()
        for b in range(B):
            kiln_amd._check(L.kiln_kv_prepare(kiln_amd._ptr(kvps[b]), kiln_amd._ptr(k[b * T:(b + 1) * T]),
                                              kiln_amd._ld(k), kiln_amd._ptr(v[b * T:(b + 1) * T]), kiln_amd._ld(v),
                                              kiln_amd._dt(k), T, H, kiln_amd._bf16_bits(kw), 1e-6,
                                              kiln_amd._ptr(rope[0]), kiln_amd._ptr(rope[1]),
                                              kiln_amd._stream(None)))

    return dict(T=T, B=B, step=step, main=main_kernel, prep=prep_only, flop=4.0 * B * H * T * T * D, q=q, k=k, v=v,
                qw=qw, kw=kw,
                rope=rope)


def linear_init(torch, out_f, in_f, g, dev):
    """torch.nn.Linear's default weight init: U(+-1/sqrt(in_features))."""
    return (torch.rand(out_f, in_f, generator=g, device=dev) * 2 - 1) / in_f ** 0.5


def context_kv(torch, kiln_amd, L, g, dev, kw, emb_dim=1024):
    """One prepared cross-attention context: N(0,1) text embeddings [L, 1024] (Qwen3-0.6B-sized) projected to
    2048 by random-init K/V weights, K RMS-normed (Dit::cache_context, engine/src/dit.cu:217-234)."""
    e = torch.randn(L, emb_dim, generator=g, device=dev)
    kk = (e @ linear_init(torch, H * D, emb_dim, g, dev).T).half()
    vv = (e @ linear_init(torch, H * D, emb_dim, g, dev).T).half()
    return kiln_amd.kv_prepare(kk, vv, H, k_norm_w=kw)


def dit_step_case(torch, kiln_amd, dev, nblocks=28, Hp=48, Wp=72, B=2, L=512, seed=100):
    """Attention of a full DiT denoising step at 768x1152 (T=3456): per block, self-attention of the CFG pair
    (QK-norm + RoPE) and cross-attention of each item against its cached context, plus the NAG negative
    attention of item 0 and the NAG combine (engine/src/dit.cu:458-488). Every block's Q/K/V and cross-attention
    Q are projections of N(0,1) activations by its own random-init 2B-shaped weights (computed at set-up, not
    timed); the three contexts (positive, unconditional, NAG negative) are projections of 1024-d embeddings,
    prepared once per generation (Dit::cache_context, engine/src/dit.cu:217-234) and outside the step."""
    T = Hp * Wp
    c, s = kiln_amd.cosmos_rope_tables(Hp, Wp)
    rope = (c.to(dev), s.to(dev))
    qw = torch.ones(D, dtype=torch.bfloat16, device=dev)  # torch RMSNorm init
    g = torch.Generator(device=dev).manual_seed(seed)
    blocks = []
    ws = torch.empty(kiln_amd.dit_self_attn_workspace_bytes(B, T, H), dtype=torch.uint8, device=dev)
    for i in range(nblocks):
        X = torch.randn(B * T, H * D, generator=g, device=dev)
        q, k, v, qc = ((X @ linear_init(torch, H * D, H * D, g, dev).T).half() for _ in range(4))
        del X
        ctx = [context_kv(torch, kiln_amd, L, g, dev, qw) for _ in range(3)]
        blocks.append((q, k, v, qc, ctx))
    a_self = torch.empty(B * T, H * D, dtype=torch.float16, device=dev)
    a_cross = torch.empty(B * T, H * D, dtype=torch.float16, device=dev)
    a_neg = torch.empty(T, H * D, dtype=torch.float16, device=dev)

    def step():
        for q, k, v, qc, ctx in blocks:
            kiln_amd.dit_self_attn(a_self, q, k, v, B, T, H, qw, qw, rope, workspace=ws)
            kiln_amd.cross_attn_nag(a_cross, qc, B, T, H, ctx[:2], [L, L], [0, 0], q_norm_w=qw, kvp_neg=ctx[2],
                                    Lk_neg=L, npad_neg=0, out_neg=a_neg)

    flop = nblocks * (4.0 * B * H * T * T * D + 4.0 * (B + 1) * H * T * L * D)
    return dict(T=T, step=step, flop=flop)


def dit_forward_case(torch, kiln_amd, dev, nblocks=28, ndistinct=4, Hp=48, Wp=72, B=2, L=512, seed=200):
    """One DiT forward of the CFG pair at config 5 on the fp16-activation path through the C++ step driver
    (kiln_amd.dit.Dit -> libkiln_dit.so, the reference's Dit::forward_batch, engine/src/dit.cu:357-546, without
    the step cache): step tables (timestep MLP + the 28 blocks' adaLN matvecs), patch embedding, 28 blocks
    (modulated LayerNorms, the Q/K/V, O, cross-Q, cross-O and MLP linear16 GEMMs with fused epilogues, fused
    self-attention, cross-attention + NAG), final layer and unpatchify. 2B shapes (D = 2048, 16 heads, MLP 8192),
    random-init bf16 weights (torch Linear's default init; 4 distinct weight sets, each block holding its own
    copy prepared at load); contexts (positive, unconditional, NAG negative, L = 512) cached outside the step.
    Also an 8-step Euler sampling run (kiln_dit_sample: the whole loop in C++)."""
    from kiln_amd import dit
    T, Dm = Hp * Wp, H * D
    g = torch.Generator(device=dev).manual_seed(seed)
    nw = torch.ones(D, dtype=torch.bfloat16, device=dev)

    def bf(o, i):
        return linear_init(torch, o, i, g, dev).to(torch.bfloat16)

    d = dit.Dit(nblocks, H, ctx_dim=1024)
    sets = []
    for _ in range(ndistinct):
        sets.append(dict(sa_q=bf(Dm, Dm), sa_k=bf(Dm, Dm), sa_v=bf(Dm, Dm), sa_o=bf(Dm, Dm), ca_q=bf(Dm, Dm),
                         ca_o=bf(Dm, Dm), ca_k=bf(Dm, 1024), ca_v=bf(Dm, 1024), mlp1=bf(4 * Dm, Dm),
                         mlp2=bf(Dm, 4 * Dm), sa_qn=nw, sa_kn=nw, ca_qn=nw, ca_kn=nw,
                         mod=[bf(256, Dm), bf(3 * Dm, 256), bf(256, Dm), bf(3 * Dm, 256), bf(256, Dm),
                              bf(3 * Dm, 256)]))
    for i in range(nblocks):
        d.set_block(i, **sets[i % ndistinct])
    del sets
    d.set_step_weights(bf(Dm, Dm), bf(3 * Dm, Dm), torch.ones(Dm, dtype=torch.bfloat16, device=dev), bf(256, Dm),
                       bf(2 * Dm, 256), bf(Dm, 68), bf(64, Dm))
    cs = [d.cache_context(torch.randn(L, 1024, generator=g, device=dev)) for _ in range(3)]
    latent = torch.randn(16, 2 * Hp, 2 * Wp, generator=g, device=dev)
    outs = [torch.empty_like(latent) for _ in range(B)]
    nag = dit.Nag(cs[2], 5.0, 2.5, 0.25)

    def step():
        d.forward(outs, latent, 0.5, cs[:2], nag=nag)

    noise = torch.randn_like(latent)
    x = torch.empty_like(latent)

    def sample8():  # 8 Euler steps, shift 3, CFG 4.5 on every step (the pair batched), NAG on the prompt item
        d.sample(x, cs[0], neg=cs[1], nag=nag, steps=8, shift=3.0, cfg=4.5, noise=noise)

    R = B * T
    gemm = 2.0 * R * Dm * Dm * 6 + 2 * 2.0 * R * 4 * Dm * Dm
    attn = 4.0 * B * H * T * T * D + 4.0 * (B + 1) * H * T * L * D
    return dict(step=step, sample8=sample8, flop=nblocks * (gemm + attn), dit=d, contexts=cs)


def linear16_cases(torch, kiln_amd, tm, dev, steps, warmup):
    """The DiT block's linear layers (kiln_linear16, fused epilogues) at config 5's CFG batch (2 x 3456 rows),
    2B model widths: Q/K/V and cross-Q (fp32 out), the two O projections (gated residual into x), MLP up (GELU,
    fp16 out) and MLP down (gated residual); torch's fp16 matmul (hipBLASLt, fp16 out, no epilogue) beside."""
    R5 = 2 * 3456
    g5 = torch.Generator(device=dev).manual_seed(55)
    xs = torch.randn(R5, 8192, device=dev, generator=g5).half()
    gate = torch.randn(8192, device=dev, generator=g5)
    lin = {}
    for name, N, K, epi in [("qkv", 2048, 2048, kiln_amd.KILN_EPI_F32), ("o_resid", 2048, 2048, kiln_amd.KILN_EPI_RESID),
                            ("mlp_up_gelu", 8192, 2048, kiln_amd.KILN_EPI_GELU16),
                            ("mlp_down_resid", 2048, 8192, kiln_amd.KILN_EPI_RESID)]:
        a = xs[:, :K].contiguous()
        w = (torch.randn(N, K, device=dev, generator=g5) * K ** -0.5).half()
        fp16_out = epi == kiln_amd.KILN_EPI_GELU16
        y = torch.zeros(R5, N, device=dev, dtype=torch.float16 if fp16_out else torch.float32)
        g = gate[:N] if epi == kiln_amd.KILN_EPI_RESID else None
        wp = kiln_amd.linear16_prepare_weight(w)  # weights are prepared once, at load
        ms_l = tm.run(lambda: kiln_amd.linear16(y, a, wp, epi=epi, gate=g), steps * 2, warmup)
        ms_p = tm.run(lambda: kiln_amd.linear16(y, a, w, epi=epi, gate=g), steps * 2, warmup)
        ms_t = tm.run(lambda: torch.matmul(a, w.t()), steps * 2, warmup)
        fl = 2.0 * R5 * N * K
        lin[name] = dict(us=ms_l * 1e3, tflops=fl / ms_l / 1e9, plain_tflops=fl / ms_p / 1e9,
                         torch_tflops=fl / ms_t / 1e9)
        log(f"linear16 {name} ({R5} x {N} x {K}): {ms_l * 1e3:.1f} us {fl / ms_l / 1e9:.1f} TFLOP/s prepared weight, "
            f"{fl / ms_p / 1e9:.1f} plain (torch fp16 matmul {fl / ms_t / 1e9:.1f})")
        del w, wp, y
    del xs
    # per DiT block: self Q, K, V and cross Q (4 x qkv), self and cross O (2 x o_resid), MLP up and down
    blk_us = 4 * lin["qkv"]["us"] + 2 * lin["o_resid"]["us"] + lin["mlp_up_gelu"]["us"] + lin["mlp_down_resid"]["us"]
    blk_fl = 2.0 * R5 * 2048 * 2048 * 6 + 2 * 2.0 * R5 * 8192 * 2048
    log(f"linear16 per DiT block: {blk_us:.1f} us {blk_fl / blk_us / 1e6:.1f} TFLOP/s")

    return lin, blk_us, blk_fl


def cpu_model():
    """The host CPU as /proc/cpuinfo names it (lscpu's "Model name"), with its family and model numbers, and the
    firmware's name for it where lscpu reports one ("BIOS Model name": a virtualized host may show only
    "AMD EPYC" in /proc/cpuinfo)."""
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                k, _, v = ln.partition(":")
                k = k.strip()
                if k in ("model name", "cpu family", "model") and k not in info:
                    info[k] = v.strip()
                if len(info) == 3:
                    break
    except OSError:
        return None
    if "model name" not in info:
        return None
    extra = ", ".join(f"{k} {info[k]}" for k in ("cpu family", "model") if k in info)
    name = f"{info['model name']} ({extra})" if extra else info["model name"]
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for ln in out.splitlines():
            k, _, v = ln.partition(":")
            if k.strip() == "BIOS Model name" and v.strip() and v.strip() != info["model name"]:
                name += f"; BIOS: {v.strip()}"
    except (OSError, ValueError, __import__("subprocess").SubprocessError):
        pass
    return name


def cpu_baseline(case, target_s=10.0):
    """The reference's fp32 two-pass attention (bench/flash_test.cu:10-32, restated in oracle/oracle.c) with
    the QK-RMSNorm and RoPE passes (kernels.cu:656-666, 759-772) on config 4: whole CFG items while they fit
    in about target_s seconds of CPU work (the full call when it does), else the first R query rows of item
    0 against all T keys."""
    import numpy as np
    import oracle
    T, B = case["T"], case["B"]
    c = case["rope"][0].cpu().numpy()
    s = case["rope"][1].cpu().numpy()
    w = case["qw"].view(__import__("torch").int16).cpu().numpy().view(np.uint16)

    def run(b, R):
        q = case["q"][b * T:b * T + R].float().cpu().numpy()
        k = case["k"][b * T:(b + 1) * T].float().cpu().numpy()
        v = case["v"][b * T:(b + 1) * T].float().cpu().numpy()
        t0 = time.perf_counter()
        qn = oracle.rope_half(oracle.rmsnorm_rows(q, w).reshape(R, H * D), H, c[:R], s[:R])
        kn = oracle.rope_half(oracle.rmsnorm_rows(k, w).reshape(T, H * D), H, c, s)
        oracle.ref_attn_f32(qn, kn, v, H)
        return time.perf_counter() - t0

    t64 = run(0, 64)
    R = int(min(T, max(64, 64 * target_s / max(t64, 1e-3))) // 64 * 64)
    dt, rows, items = run(0, R), R, 1
    while R == T and items < B and dt * (items + 1) / items <= 1.5 * target_s:
        dt += run(items, T)
        rows += T
        items += 1
    flop = 4.0 * rows * H * T * D
    what = (f"config 4, {items} of {B} CFG items in full" if R == T else f"config 4 item 0: {R} of {T} query rows")
    return dict(value=round(flop / dt / 1e12, 5), unit="TFLOP/s", cores=oracle.num_threads(), kind="port",
                nproc=os.cpu_count(), cpu_model=cpu_model(),
                sample=f"{what} x {H} heads x {T} keys (+ QK-RMSNorm, RoPE), fp32 two-pass reference attention, "
                       f"{dt:.1f} s")


def cpu_baseline_configs():
    """The same CPU reference (the fp32 two-pass attention of bench/flash_test.cu:10-32 with the QK-RMSNorm and
    RoPE passes and the NAG combine of engine/src/dit.cu:295-324, all from oracle/oracle.c) on configs 1-3 in
    full and on one of config 5's 28 blocks (its self-attention of the CFG pair, the cross-attention of both
    items and the NAG negative attention of item 0 over L = 512, and the NAG combine), scaled by 28 to a step.
    Inputs are seeded N(0,1) rows of each config's shapes (the CPU time does not depend on the values); Q/K
    norm weights 1 (torch's RMSNorm init)."""
    import numpy as np
    import oracle
    rng = np.random.default_rng(7)

    def randn(*shape):
        return rng.standard_normal(shape, dtype=np.float32)

    w1 = np.full(D, 0x3F80, np.uint16)  # bf16 1.0

    def normed_roped(x, c, s):
        return oracle.rope_half(oracle.rmsnorm_rows(x, w1).reshape(x.shape[0], H * D), H, c, s)

    def timed(fn):
        t0 = time.perf_counter()
        fn()
        return time.perf_counter() - t0

    out = {}
    # config 1: plain self-attention, S = 1536, B = 1
    q, k, v = randn(1536, H * D), randn(1536, H * D), randn(1536, H * D)
    dt = timed(lambda: oracle.ref_attn_f32(q, k, v, H))
    fl = 4.0 * H * 1536 * 1536 * D
    out["config1"] = dict(tflops=round(fl / dt / 1e12, 5), seconds=round(dt, 3),
                          sample="in full: B=1, S=1536, 16 heads, fp32 two-pass reference attention")
    # config 2: the CFG pair at T = 1536 with QK-RMSNorm and RoPE
    c2, s2 = (t.numpy() for t in __import__("kiln_amd").cosmos_rope_tables(32, 48))
    qs, ks, vs = ([randn(1536, H * D) for _ in range(2)] for _ in range(3))
    dt = timed(lambda: [oracle.ref_attn_f32(normed_roped(qs[b], c2, s2), normed_roped(ks[b], c2, s2), vs[b], H)
                        for b in range(2)])
    fl = 2 * 4.0 * H * 1536 * 1536 * D
    out["config2"] = dict(tflops=round(fl / dt / 1e12, 5), seconds=round(dt, 3),
                          sample="in full: B=2, T=1536, 16 heads, QK-RMSNorm + RoPE + fp32 two-pass attention")
    # config 3: cross-attention over a positive and a negative context of 512 keys, NAG combine
    q3 = oracle.rmsnorm_rows(randn(1536, H * D), w1).reshape(1536, H * D)
    kp, vp, kn, vn = (randn(512, H * D) for _ in range(4))

    def cfg3():
        zp = oracle.ref_attn_f32(q3, kp, vp, H)
        zn = oracle.ref_attn_f32(q3, kn, vn, H)
        oracle.nag(zp, zn)

    dt = timed(cfg3)
    fl = 2 * 4.0 * H * 1536 * 512 * D
    out["config3"] = dict(tflops=round(fl / dt / 1e12, 5), seconds=round(dt, 3),
                          sample="in full: 1536 queries x (positive + negative) 512-key contexts, 16 heads, NAG")
    # config 5: one block of 28 (T = 3456, B = 2, L = 512), scaled to the step
    T5, L5 = 3456, 512
    c5, s5 = (t.numpy() for t in __import__("kiln_amd").cosmos_rope_tables(48, 72))
    qs, ks, vs, qc = ([randn(T5, H * D) for _ in range(2)] for _ in range(4))
    ctx = [(randn(L5, H * D), randn(L5, H * D)) for _ in range(3)]

    def block():
        for b in range(2):
            oracle.ref_attn_f32(normed_roped(qs[b], c5, s5), normed_roped(ks[b], c5, s5), vs[b], H)
        qn = [oracle.rmsnorm_rows(qc[b], w1).reshape(T5, H * D) for b in range(2)]
        z0 = oracle.ref_attn_f32(qn[0], *ctx[0], H)
        oracle.ref_attn_f32(qn[1], *ctx[1], H)
        zn = oracle.ref_attn_f32(qn[0], *ctx[2], H)
        oracle.nag(z0, zn)

    dt = timed(block)
    fl = 4.0 * 2 * H * T5 * T5 * D + 4.0 * 3 * H * T5 * L5 * D
    out["config5"] = dict(tflops=round(fl / dt / 1e12, 5), ms_per_step=round(28 * dt * 1e3, 1), seconds=round(dt, 3),
                          sample="block 0 of 28 in full (self-attention of the CFG pair with QK-RMSNorm + RoPE, "
                                 "cross-attention of both items and the NAG negative over 512 keys, NAG combine), "
                                 "x 28 for the step")
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--main-only", action="store_true",
                    help="run only the config-4 attention kernel loop, back to back (for rocprofv3 runs)")
    ap.add_argument("--call-only", action="store_true",
                    help="run only the config-4 whole call (K/V prepare + attention) loop (for rocprofv3 runs)")
    ap.add_argument("--linear16-only", action="store_true",
                    help="run only the DiT-shape linear16 cases (for rocprofv3 runs)")
    ap.add_argument("--forward-only", action="store_true",
                    help="run only the config-5 DiT forward of the CFG pair (for rocprofv3 runs)")
    ap.add_argument("--copy-cal", type=int, default=0, metavar="MIB",
                    help="copy a MIB-sized device buffer --steps times (calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the path has no "
              f"collective and shards by head with no communication, so run with --gpus 1.", file=sys.stderr)
        return 2

    import torch
    import kiln_amd
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    dev = "cuda:0"
    torch.cuda.set_device(0)
    L = kiln_amd.lib()  # fails loudly when the HIP library is missing
    buf = __import__("ctypes").create_string_buffer(64)
    L.kiln_attn_device_arch(0, buf, 64)
    arch = buf.value.decode()
    tm = Timer(torch)
    if args.copy_cal:
        src = torch.empty(args.copy_cal << 18, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        ms = tm.run(lambda: dst.copy_(src), args.steps, args.warmup)
        log(f"copy {args.copy_cal} MiB: {ms * 1e3:.1f} us  {2 * src.numel() * 4 / ms / 1e6:.1f} GB/s")
        return 0

    if args.linear16_only:
        linear16_cases(torch, kiln_amd, tm, dev, args.steps, args.warmup)
        return 0
    if args.forward_only:
        cf = dit_forward_case(torch, kiln_amd, dev)
        ms = tm.run(cf["step"], args.steps, args.warmup)
        log(f"config 5 DiT forward of the CFG pair: {ms:.3f} ms")
        return 0

    cfg4 = self_attn_case(torch, kiln_amd, 64, 64, 2, 4, dev)
    if args.main_only or args.call_only:
        ms = tm.run(cfg4["main" if args.main_only else "step"], args.steps, args.warmup)
        log(f"{'k_attn_fwd' if args.main_only else 'whole call'} config 4: {ms * 1e3:.1f} us  "
            f"{cfg4['flop'] / ms / 1e9:.1f} TFLOP/s")
        return 0

    ms4 = tm.run(cfg4["step"], args.steps, args.warmup)
    # the dominant kernel's duration inside the call (prepare -> attention, events around the attention launch),
    # and back to back without the prepare pass
    ms4_main = tm.run_inner(cfg4["prep"], cfg4["main"], args.steps, args.warmup)
    ms4_alone = tm.run(cfg4["main"], args.steps, args.warmup)
    tf4 = cfg4["flop"] / ms4 / 1e9
    tf4_main = cfg4["flop"] / ms4_main / 1e9
    log(f"config 4 (T=4096, B=2): {ms4 * 1e3:.1f} us/call  {tf4:.1f} TFLOP/s  ({tf4 / PEAK_TFLOPS * 100:.1f}% peak); "
        f"attention kernel inside the call {ms4_main * 1e3:.1f} us  {tf4_main:.1f} TFLOP/s, back to back "
        f"{ms4_alone * 1e3:.1f} us")

    # one GPU's share of config 4 under 8-way head (tensor) parallelism: H = 2 of the 16 heads, same call
    # (the first two heads of the same tensors); 128 workgroups, a quarter of the resident slots
    h8 = 2
    out8 = torch.empty_like(cfg4["q"])
    ws8 = torch.empty(kiln_amd.dit_self_attn_workspace_bytes(2, cfg4["T"], h8), dtype=torch.uint8, device=dev)
    ms_tp = tm.run(lambda: kiln_amd.dit_self_attn(out8, cfg4["q"], cfg4["k"], cfg4["v"], 2, cfg4["T"], h8, cfg4["qw"],
                                                  cfg4["kw"], cfg4["rope"], workspace=ws8), args.steps, args.warmup)
    tf_tp = cfg4["flop"] * h8 / H / ms_tp / 1e9
    log(f"config 4, one GPU's share of 8-way head parallelism (H=2): {ms_tp * 1e3:.1f} us/call  {tf_tp:.1f} TFLOP/s")
    del out8, ws8

    # the unchanged-engine drop-in: attention16() with fp32 Q/K/V (already normed and roped, as the reference
    # engine hands them over, engine/src/dit.cu:464-469), one call per CFG item at config 4's shape
    qf, kf, vf = (t[:cfg4["T"]].float() for t in (cfg4["q"], cfg4["k"], cfg4["v"]))
    o16 = torch.empty(cfg4["T"], H * D, dtype=torch.float16, device=dev)
    ms_di = tm.run(lambda: kiln_amd.attention16(o16, qf, kf, vf, cfg4["T"], cfg4["T"], H), args.steps, args.warmup)
    tf_di = cfg4["flop"] / 2 / ms_di / 1e9
    log(f"drop-in attention16 (fp32 Q/K/V, one CFG item of config 4): {ms_di * 1e3:.1f} us/call  {tf_di:.1f} TFLOP/s")
    del qf, kf, vf, o16

    cfg2 = self_attn_case(torch, kiln_amd, 32, 48, 2, 2, dev)
    ms2 = tm.run(cfg2["step"], args.steps, args.warmup)
    tf2 = cfg2["flop"] / ms2 / 1e9
    log(f"config 2 (T=1536, B=2): {ms2 * 1e3:.1f} us/call  {tf2:.1f} TFLOP/s  ({tf2 / PEAK_TFLOPS * 100:.1f}% peak)")
    del cfg2

    # config 3: text cross-attention with NAG, 1536 queries (projected, RMS-normed in the call) over a positive
    # and a negative 512-token context (1024-d embeddings projected to 2048, prepared once per generation,
    # outside the call), NAG combine of the two outputs
    T3, L3 = 1536, 512
    g3 = torch.Generator(device=dev).manual_seed(3)
    q3 = (torch.randn(T3, H * D, generator=g3, device=dev) @ linear_init(torch, H * D, H * D, g3, dev).T).half()
    w3 = torch.ones(D, dtype=torch.bfloat16, device=dev)
    ctx3 = [context_kv(torch, kiln_amd, L3, g3, dev, w3) for _ in range(2)]
    o3 = torch.empty(T3, H * D, dtype=torch.float16, device=dev)
    n3 = torch.empty(T3, H * D, dtype=torch.float16, device=dev)
    ms3 = tm.run(lambda: kiln_amd.cross_attn_nag(o3, q3, 1, T3, H, ctx3[:1], [L3], [0], q_norm_w=w3, kvp_neg=ctx3[1],
                                                 Lk_neg=L3, npad_neg=0, out_neg=n3), args.steps, args.warmup)
    tf3 = 2 * 4.0 * H * T3 * L3 * D / ms3 / 1e9
    log(f"config 3 (cross-attention 1536 x 512, positive + negative + NAG): {ms3 * 1e3:.1f} us/call  {tf3:.1f} TFLOP/s")
    del q3, ctx3, o3, n3

    cfg5 = dit_step_case(torch, kiln_amd, dev)
    ms5 = tm.run(cfg5["step"], max(3, args.steps // 4), max(1, args.warmup // 2))
    log(f"config 5 (T=3456, 28 blocks, self + cross + NAG): {ms5:.3f} ms attention per DiT step  "
        f"{cfg5['flop'] / ms5 / 1e9:.1f} TFLOP/s")
    del cfg5

    # the DiT block's HBM-bound passes around attention at config 5's CFG batch (2 x 3456 rows x 2048):
    # modulated LayerNorm to fp16 (read 4 B, write 2 B per element) and the gated residual (read 8, write 4)
    R5 = 2 * 3456
    x5 = torch.randn(R5, H * D, device=dev)
    y5 = torch.randn(R5, H * D, device=dev)
    sc5, sh5 = torch.randn(H * D, device=dev) * 0.1, torch.randn(H * D, device=dev)
    n16 = torch.empty(R5, H * D, dtype=torch.float16, device=dev)
    ms_ln = tm.run(lambda: kiln_amd.layernorm_mod(n16, x5, sc5, sh5), args.steps * 5, args.warmup)
    ms_ag = tm.run(lambda: kiln_amd.add_gated(x5, y5, sc5), args.steps * 5, args.warmup)
    ln_tbps = 6.0 * R5 * H * D / ms_ln / 1e9
    ag_tbps = 12.0 * R5 * H * D / ms_ag / 1e9
    log(f"layernorm_mod16 (6912 x 2048): {ms_ln * 1e3:.1f} us {ln_tbps:.2f} TB/s; add_gated: {ms_ag * 1e3:.1f} us "
        f"{ag_tbps:.2f} TB/s")
    del x5, y5, n16

    lin, blk_us, blk_fl = linear16_cases(torch, kiln_amd, tm, dev, args.steps, args.warmup)

    # the self-attention section of one DiT block at config 5 from the fp16 LayerNorm output: fused (QKV GEMM
    # epilogue does QK-norm + RoPE + K/V preparation, then attention) against unfused (fp32 QKV GEMM, then the
    # fused attention call with its K/V prepare pass)
    T5, D5 = 3456, H * D
    g6 = torch.Generator(device=dev).manual_seed(66)
    x16 = torch.randn(2 * T5, D5, generator=g6, device=dev).half()
    wqkv = kiln_amd.linear16_prepare_weight(linear_init(torch, 3 * D5, D5, g6, dev).half())
    nw5 = torch.ones(D, dtype=torch.bfloat16, device=dev)
    c5, s5 = kiln_amd.cosmos_rope_tables(48, 72)
    rope5 = (c5.to(dev), s5.to(dev))
    a5 = torch.empty(2 * T5, D5, dtype=torch.float16, device=dev)
    ws5 = torch.empty(L.kiln_dit_self_attn_x16_workspace_bytes(2, T5, H), dtype=torch.uint8, device=dev)
    qkv5 = torch.empty(2 * T5, 3 * D5, device=dev)
    wsu = torch.empty(kiln_amd.dit_self_attn_workspace_bytes(2, T5, H), dtype=torch.uint8, device=dev)
    ms_fz = tm.run(lambda: kiln_amd.dit_self_attn_x16(a5, x16, wqkv, 2, T5, H, nw5, nw5, rope5, workspace=ws5),
                   args.steps, args.warmup)

    def unfused():
        kiln_amd.linear16(qkv5, x16, wqkv)
        kiln_amd.dit_self_attn(a5, qkv5[:, :D5], qkv5[:, D5:2 * D5], qkv5[:, 2 * D5:], 2, T5, H, nw5, nw5, rope5,
                               workspace=wsu)

    ms_uf = tm.run(unfused, args.steps, args.warmup)
    log(f"config 5 self-attention section from x16 (QKV GEMM + attention): fused epilogue {ms_fz * 1e3:.1f} us, "
        f"unfused {ms_uf * 1e3:.1f} us")
    del x16, wqkv, a5, ws5, qkv5, wsu

    cfgb = dit_forward_case(torch, kiln_amd, dev)
    ms_blk = tm.run(cfgb["step"], max(3, args.steps // 5), 1)
    # the same forward's attention on the production path (QKV projection epilogue preparing K/V, 28 blocks of
    # self-attention of the pair + cross-attention + NAG), from the library's per-category event timing
    kiln_amd.prof_enable(True)
    cfgb["step"]()
    cats, _ = kiln_amd.prof_report()
    kiln_amd.prof_enable(False)
    ms5_fused = cats.get("attention", (float("nan"), 0))[0]
    log(f"config 5, attention of the fused-path forward (profiler): {ms5_fused:.3f} ms over "
        f"{cats.get('attention', (0, 0))[1]} calls; GEMMs {cats.get('gemm_tc16', (0, 0))[0]:.3f} ms")
    log(f"config 5, DiT forward of the CFG pair on the fp16 path (step tables, embed, 28 blocks, final layer): "
        f"{ms_blk:.3f} ms per step  {cfgb['flop'] / ms_blk / 1e9:.1f} TFLOP/s")
    cfgb_flop = cfgb["flop"]
    ms_s8 = tm.run(cfgb["sample8"], 2, 1)
    log(f"config 5, 8-step Euler sampling with CFG 4.5 + NAG (8 forwards of the CFG pair): {ms_s8:.1f} ms")
    # the fp32 branch of the same forward (the reference's "precision": "fp32" jobs: fp32 linears, RMSNorm, RoPE,
    # exact fp32 attention), contexts cached for it
    from kiln_amd import dit as _dit
    g32 = torch.Generator(device=dev).manual_seed(32)
    cs32 = [cfgb["dit"].cache_context(torch.randn(512, 1024, generator=g32, device=dev), fp32=True) for _ in range(3)]
    lat32 = torch.randn(16, 96, 144, generator=g32, device=dev)
    outs32 = [torch.empty_like(lat32) for _ in range(2)]
    nag32 = _dit.Nag(cs32[2], 5.0, 2.5, 0.25)
    ms_f32 = tm.run(lambda: cfgb["dit"].forward(outs32, lat32, 0.5, cs32[:2], nag=nag32, fp32=True), 2, 1)
    log(f"config 5, DiT forward of the CFG pair on the fp32 path: {ms_f32:.1f} ms per step")
    del cs32, outs32, nag32
    del cfgb

    # HBM bytes per launch of k_attn_fwd (config 4): the committed rocprofv3 FETCH_SIZE / WRITE_SIZE runs, with the
    # commit whose kernel they measured
    traffic, traffic_commit = None, None
    tpath = os.path.join(ROOT, "profiles", "k_attn_fwd_config4_hbm_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            tj = json.load(f)
        traffic, traffic_commit = tj.get("traffic_bytes"), tj.get("commit")

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(cfg4)
        cpu["configs"] = cpu_baseline_configs()
        log(f"cpu baseline: {cpu}")

    line = {
        "metric": METRIC,
        "value": round(tf4, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms4, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: N(0,1) activations x random-init (torch Linear) projection weights, seeded",
        "config": {
            "workload": "config 4: DiT self-attention 1024x1024 (T=4096), CFG batch 2, H=16, d=128, fp16 Q/K/V, "
                        "QK-RMSNorm + 3D RoPE fused; step = K/V prepare + attention",
            "arch": arch,
            "pct_fp16_peak": round(tf4 / PEAK_TFLOPS * 100, 2),
            "attention_kernel_in_call_us": round(ms4_main * 1e3, 2),
            "attention_kernel_back_to_back_us": round(ms4_alone * 1e3, 2),
            "dropin_attention16_f32in_ms_per_call": round(ms_di, 5),
            "dropin_attention16_f32in_tflops": round(tf_di, 2),
            "tp8_share_h2_ms_per_call": round(ms_tp, 5),
            "tp8_share_h2_tflops": round(tf_tp, 2),
            "s1536_tflops": round(tf2, 2),
            "s1536_pct_fp16_peak": round(tf2 / PEAK_TFLOPS * 100, 2),
            "s1536_ms_per_call": round(ms2, 5),
            "cross_nag_1536x512_ms_per_call": round(ms3, 5),
            "cross_nag_1536x512_tflops": round(tf3, 2),
            "dit_step_attention_ms": round(ms5, 4),
            "dit_step_attention_ms_fused_path": round(ms5_fused, 4),
            "dit_step_workload": "config 5: 768x1152 (T=3456), B=2, 28 blocks x (self + cross L=512 + NAG)",
            "layernorm_mod16_us": round(ms_ln * 1e3, 2),
            "layernorm_mod16_tbps": round(ln_tbps, 3),
            "add_gated_us": round(ms_ag * 1e3, 2),
            "add_gated_tbps": round(ag_tbps, 3),
            "linear16_tflops": {k: round(v["tflops"], 1) for k, v in lin.items()},
            "linear16_plain_weight_tflops": {k: round(v["plain_tflops"], 1) for k, v in lin.items()},
            "linear16_torch_f16out_tflops": {k: round(v["torch_tflops"], 1) for k, v in lin.items()},
            "linear16_dit_block_us": round(blk_us, 1),
            "linear16_dit_block_tflops": round(blk_fl / blk_us / 1e6, 1),
            "dit_self_attn_section_fused_us": round(ms_fz * 1e3, 1),
            "dit_self_attn_section_unfused_us": round(ms_uf * 1e3, 1),
            "dit_forward_ms_per_step": round(ms_blk, 3),
            "dit_forward_tflops": round(cfgb_flop / ms_blk / 1e9, 1),
            "dit_sample_8_steps_ms": round(ms_s8, 1),
            "dit_forward_fp32_path_ms_per_step": round(ms_f32, 1),
            "dit_forward_workload": "config 5: Dit::forward_batch of the CFG pair on the fp16 path (step tables, patch "
                                    "embed, 28 x (3 LN16 + Q/K/V, O, cross-Q, cross-O, MLP linear16 + self-attn + "
                                    "cross-attn L=512 + NAG), final layer), B=2, T=3456, 2B shapes",
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "k_attn_fwd",
            "achieved": round(tf4_main, 2),
            "peak": PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(tf4_main / PEAK_TFLOPS, 4),
            "traffic": traffic,
            "traffic_source": "profiles/k_attn_fwd_config4_hbm_traffic.md",
            "traffic_commit": traffic_commit,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
