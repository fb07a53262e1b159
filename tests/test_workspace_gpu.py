"""The drop-ins' workspace modes (include/kiln_attn.h): once reserved, a drop-in call allocates nothing and never
synchronizes, so it can be captured into a HIP graph; a call that needs more than the reservation fails with
KILN_ENOMEM instead of growing it. The reference's flash paths take their scratch from the engine's arena and
allocate nothing per call (engine/src/kernels.cu:828-873, gpu.h:51-59)."""
import ctypes

import numpy as np
import pytest
import torch

import kiln_amd
from kiln_amd import KILN_ENOMEM, KilnError

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
H, D = 16, 128


def _inputs(seed, Tq, Tk):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(Tq, H * D, generator=g).to(DEV)
    k = torch.randn(Tk, H * D, generator=g).to(DEV)
    v = torch.randn(Tk, H * D, generator=g).to(DEV)
    return q, k, v


def test_dropin_reserved_workspace_graph_capture(gpu):
    L = gpu
    Tq = Tk = 1024
    q, k, v = _inputs(5, Tq, Tk)
    eager = torch.empty(Tq, H * D, dtype=torch.float16, device=DEV)
    kiln_amd.attention16(eager, q, k, v, Tq, Tk, H)
    torch.cuda.synchronize()
    need = L.kiln_attn_dropin_workspace_bytes(Tq, Tk, H)
    assert need >= kiln_amd.kv_prepped_bytes(Tk, H)
    assert L.kiln_attn_workspace_release() == 0  # drop what earlier calls grew, so the reservation is exactly need
    assert L.kiln_attn_workspace_reserve(need) == 0
    try:
        out = torch.empty_like(eager)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):  # any hipMalloc or device synchronize inside would fail the capture
            kiln_amd.attention16(out, q, k, v, Tq, Tk, H)
        for rep in range(3):
            out.fill_(float("nan"))  # the program's own eager work between replays
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"replay {rep} differs from the eager call"
        # beyond the reservation: an error, not a larger allocation
        q2, k2, v2 = _inputs(6, Tq, 2 * Tk)
        with pytest.raises(KilnError) as ei:
            kiln_amd.attention16(out, q2, k2, v2, Tq, 2 * Tk, H)
        assert ei.value.status == KILN_ENOMEM
        del graph
    finally:
        torch.cuda.synchronize()
        assert L.kiln_attn_workspace_release() == 0


def test_dropin_bound_workspace(gpu):
    """A caller-owned buffer bound with kiln_attn_set_workspace (the engine's arena) gives the same results."""
    L = gpu
    Tq, Tk = 700, 900
    q, k, v = _inputs(7, Tq, Tk)
    ref = torch.empty(Tq, H * D, dtype=torch.float32, device=DEV)
    kiln_amd.attention(ref, q, k, v, Tq, Tk, H)
    need = L.kiln_attn_dropin_workspace_bytes(Tq, Tk, H)
    arena = torch.empty(need + 4096, dtype=torch.uint8, device=DEV)
    base = (arena.data_ptr() + 255) // 256 * 256
    torch.cuda.synchronize()
    assert L.kiln_attn_set_workspace(ctypes.c_void_p(base), need) == 0
    try:
        out = torch.empty_like(ref)
        kiln_amd.attention(out, q, k, v, Tq, Tk, H)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
    finally:
        assert L.kiln_attn_set_workspace(None, 0) == 0
    assert np.isfinite(out.cpu().numpy()).all()
