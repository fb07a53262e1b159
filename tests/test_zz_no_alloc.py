"""kiln_attn_fwd_f16out_noalloc (attention16 on the library's fixed device scratch, for callers that cannot
allocate) against kiln_attn_fwd_f16out on the same inputs: bit-identical outputs, on two calls in a row, the
second one smaller (the scratch keeps the first call's contents; nothing may depend on them)."""
import ctypes

import pytest
import torch

import kiln_amd

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
H, D = 16, 128
_vp = ctypes.c_void_p


def _fn(L):
    return L.kiln_attn_fwd_f16out_noalloc  # argument types bound by kiln_amd.lib()


def _call(f, out, q, k, v, Tq, Tk, npad):
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return f(_vp(out.data_ptr()), out.stride(0), _vp(q.data_ptr()), q.stride(0), _vp(k.data_ptr()), k.stride(0),
             _vp(v.data_ptr()), v.stride(0), Tq, Tk, H, D, npad, s)


@pytest.mark.parametrize("shapes", [((1536, 1536, 0), (300, 700, 5)), ((4096, 4096, 0), (128, 2000, 0))])
def test_noalloc_matches_allocating_entry_point(gpu, shapes):
    f = _fn(gpu)
    assert gpu.kiln_attn_noalloc_scratch_bytes() == 64 << 20
    for n, (Tq, Tk, npad) in enumerate(shapes):
        print(f"[noalloc] call {n}: Tq={Tq} Tk={Tk} npad={npad}", flush=True)
        g = torch.Generator().manual_seed(100 + n)
        q, k, v = (torch.randn(T, H * D, generator=g).to(DEV) for T in (Tq, Tk, Tk))
        ref = torch.full((Tq, H * D), float("nan"), dtype=torch.float16, device=DEV)
        got = torch.full_like(ref, float("nan"))
        kiln_amd.attention16(ref, q, k, v, Tq, Tk, H, npad=npad)
        assert _call(f, got, q, k, v, Tq, Tk, npad) == 0, gpu.kiln_attn_last_error().decode()
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got, ref), f"call {n}: no-alloc output differs from kiln_attn_fwd_f16out"


def test_noalloc_rejects_beyond_scratch(gpu):
    f = _fn(gpu)
    Tk = 9000  # 16 heads x 141 tiles x 32 KB > 64 MiB
    q = torch.zeros(8, H * D, device=DEV)
    kv = torch.zeros(Tk, H * D, device=DEV)
    out = torch.empty(8, H * D, dtype=torch.float16, device=DEV)
    assert _call(f, out, q, kv, kv, 8, Tk, 0) == kiln_amd.KILN_ENOMEM
    assert b"scratch" in gpu.kiln_attn_last_error()


def test_noalloc_orders_calls_on_two_streams(gpu):
    """Two streams alternate calls on the shared scratch without any host synchronization in between: the entry
    point makes each call wait for the previous call on the other stream, so every output equals the allocating
    entry point's (a long call is followed at once by a short one on the other stream)."""
    f = _fn(gpu)
    shapes = [(4096, 4096, 0), (200, 300, 3), (2048, 3000, 0), (64, 4000, 0)]
    ins, refs = [], []
    for n, (Tq, Tk, npad) in enumerate(shapes):
        g = torch.Generator().manual_seed(300 + n)
        q, k, v = (torch.randn(T, H * D, generator=g).to(DEV) for T in (Tq, Tk, Tk))
        ref = torch.empty(Tq, H * D, dtype=torch.float16, device=DEV)
        kiln_amd.attention16(ref, q, k, v, Tq, Tk, H, npad=npad)
        ins.append((q, k, v))
        refs.append(ref)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [torch.full((T, H * D), float("nan"), dtype=torch.float16, device=DEV) for T, _, _ in shapes]
    torch.cuda.synchronize()
    for rep in range(3):
        for n, (Tq, Tk, npad) in enumerate(shapes):
            s = streams[n % 2]
            print(f"[noalloc] two streams: rep {rep} call {n} Tq={Tq} Tk={Tk}", flush=True)
            with torch.cuda.stream(s):
                q, k, v = ins[n]
                assert _call(f, outs[n], q, k, v, Tq, Tk, npad) == 0, gpu.kiln_attn_last_error().decode()
        torch.cuda.synchronize()
        for n in range(len(shapes)):
            assert torch.equal(outs[n], refs[n]), f"rep {rep} call {n}: output differs from the allocating path"
