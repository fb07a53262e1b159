"""The C-ABI library on the CPU: it loads, exports every symbol include/kiln_attn.h declares, and its
host-side logic (status strings, argument validation that returns before any HIP call, buffer sizes, the
host Cosmos RoPE tables) behaves as documented. No kernel is launched here."""
import ctypes

import numpy as np
import pytest

import kiln_amd
import oracle


@pytest.fixture(scope="module")
def L():
    return kiln_amd.lib()


def test_exports_every_header_symbol(L):
    syms = kiln_amd.header_symbols()
    assert len(syms) >= 18
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, f"declared in include/kiln_attn.h but not exported: {missing}"
    # every declared symbol is bound with a signature in the Python mirror, and nothing else is
    assert sorted(kiln_amd._SIGS) == syms


def test_status_strings(L):
    for code in range(5):
        assert L.kiln_attn_status_string(code).decode()
    assert L.kiln_attn_status_string(99).decode() == "unknown status"


def test_kv_prepped_bytes(L):
    # [H][ceil(Tk/64)][K 16 KB | V 16 KB]
    assert L.kiln_kv_prepped_bytes(1, 16) == 16 * 1 * 32768
    assert L.kiln_kv_prepped_bytes(64, 16) == 16 * 1 * 32768
    assert L.kiln_kv_prepped_bytes(65, 2) == 2 * 2 * 32768
    assert L.kiln_kv_prepped_bytes(4096, 16) == 16 * 64 * 32768
    assert L.kiln_kv_prepped_bytes(0, 16) == 0
    assert L.kiln_dit_self_attn_workspace_bytes(2, 4096, 16) == 2 * L.kiln_kv_prepped_bytes(4096, 16)


def test_cosmos_rope_tables_host_equal_oracle(L):
    """kiln_cosmos_rope_tables is host code in the library (engine/src/dit.cu:196-215): bitwise equal to the
    oracle's restatement, which tests/test_oracle.py pins against the float64 Cosmos formulas."""
    for Hp, Wp in ((32, 48), (64, 64), (48, 72)):
        c = np.empty((Hp * Wp, 64), np.float32)
        s = np.empty((Hp * Wp, 64), np.float32)
        assert L.kiln_cosmos_rope_tables(c.ctypes.data, s.ctypes.data, Hp, Wp) == 0
        oc, os_ = oracle.cosmos_rope(Hp, Wp)
        np.testing.assert_array_equal(c, oc)
        np.testing.assert_array_equal(s, os_)
    assert L.kiln_cosmos_rope_tables(None, None, 4, 4) == kiln_amd.KILN_EINVAL


def test_argument_validation_without_gpu(L):
    """Checks that reject a call before any HIP call (the reference throws on the same shapes)."""
    p = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation first
    # attention16 needs Dh = 128 (engine/src/kernels.cu:870)
    assert L.kiln_attn_fwd_f16out(p, 1024, p, 1024, p, 1024, p, 1024, 8, 8, 16, 64, 0, None) == kiln_amd.KILN_EUNSUPPORTED
    assert "head size" in L.kiln_attn_last_error().decode()
    # no keys at all: softmax undefined
    assert L.kiln_attn_fwd_f32out(p, 2048, p, 2048, p, 2048, p, 2048, 8, 0, 16, 128, 0, 0, None) == kiln_amd.KILN_EINVAL
    # negative sizes
    assert L.kiln_attn_fwd_f32out(p, 2048, p, 2048, p, 2048, p, 2048, -1, 8, 16, 128, 0, 0, None) == kiln_amd.KILN_EINVAL
    # flash path: 32-bit buffer offsets bound the keys per head
    assert L.kiln_attn_fwd_f32out(p, 2048, p, 2048, p, 2048, p, 2048, 8, (1 << 22) + 1, 16, 128, 0, 0, None) == \
        kiln_amd.KILN_EUNSUPPORTED
    assert L.kiln_kv_prepare(p, p, 2048, p, 2048, 1, (1 << 22) + 1, 16, None, 1e-6, None, None, None) == \
        kiln_amd.KILN_EUNSUPPORTED
    # exact path: head size bound
    assert L.kiln_attn_fwd_exact(p, 4096, p, 4096, p, 4096, p, 4096, 8, 8, 8, 512, 0, 0, None) == kiln_amd.KILN_EUNSUPPORTED
    # dtype codes
    assert L.kiln_nag_combine(p, 8, p, 8, 7, 4, 8, 5.0, 2.5, 0.25, None) == kiln_amd.KILN_EINVAL
    assert L.kiln_kv_prepare(p, p, 2048, p, 2048, 3, 64, 16, None, 1e-6, None, None, None) == kiln_amd.KILN_EINVAL
    # modulated LayerNorm / gated residual: sizes and null pointers
    assert L.kiln_layernorm_mod(p, p, p, p, 4, 0, 1e-6, None) == kiln_amd.KILN_EINVAL
    assert L.kiln_layernorm_mod16(p, p, None, p, 4, 2048, 1e-6, None) == kiln_amd.KILN_EINVAL
    assert L.kiln_add_gated(p, None, None, 4, 2048, None) == kiln_amd.KILN_EINVAL
    assert L.kiln_add_gated(p, p, None, -1, 2048, None) == kiln_amd.KILN_EINVAL
    # linear16: the reference's eligibility (tcgemm16.cuh:177), epilogue code, alignment, output stride
    q = ctypes.c_void_p(4096)
    assert L.kiln_linear16(q, 128, q, 8, q, 128, 40, 0, None, 0.0, None, None, 0, None) == kiln_amd.KILN_EUNSUPPORTED
    assert L.kiln_linear16(q, 128, q, 8, q, 96, 64, 0, None, 0.0, None, None, 0, None) == kiln_amd.KILN_EUNSUPPORTED
    assert L.kiln_linear16(q, 128, q, 8, q, 128, 64, 0, None, 0.0, q, q, 16, None) == kiln_amd.KILN_EUNSUPPORTED
    assert L.kiln_linear16(q, 128, q, 8, q, 128, 64, 4, None, 0.0, None, None, 0, None) == kiln_amd.KILN_EINVAL
    assert L.kiln_linear16(q, 64, q, 8, q, 128, 64, 0, None, 0.0, None, None, 0, None) == kiln_amd.KILN_EINVAL
    assert L.kiln_linear16(q, 128, ctypes.c_void_p(4104), 8, q, 128, 64, 0, None, 0.0, None, None, 0, None) == \
        kiln_amd.KILN_EUNSUPPORTED
    assert L.kiln_linear16(q, 129, q, 8, q, 128, 64, 0, None, 0.0, None, None, 0, None) == kiln_amd.KILN_EUNSUPPORTED
    assert L.kiln_linear16(q, 128, None, 8, q, 128, 64, 0, None, 0.0, None, None, 0, None) == kiln_amd.KILN_EINVAL
    assert L.kiln_linear16(None, 128, None, 0, None, 128, 64, 0, None, 0.0, None, None, 0, None) == kiln_amd.KILN_OK
    # prepared weights: size, eligibility, overlap
    assert L.kiln_linear16_prepped_weight_bytes(384, 64) == 512 * 64 * 2
    assert L.kiln_linear16_prepped_weight_bytes(0, 64) == 0
    assert L.kiln_linear16_prepare_weight(q, q, 96, 64, 0, None) == kiln_amd.KILN_EUNSUPPORTED
    assert L.kiln_linear16_prepare_weight(q, ctypes.c_void_p(4096 + 1024), 128, 64, 0, None) == kiln_amd.KILN_EINVAL
    assert L.kiln_linear16_prepare_weight(None, q, 128, 64, 0, None) == kiln_amd.KILN_EINVAL
    assert L.kiln_linear16_prepped(q, 128, q, 8, q, 128, 40, 0, None, 0.0, None, None, 0, None) == kiln_amd.KILN_EUNSUPPORTED
    # fused-projection DiT sections: odd H, batch bound, workspace too small, null pointers
    assert L.kiln_dit_self_attn_x16(q, 1, 384, q, q, q, q, 1e-6, q, q, 2, 96, 3, q, 1 << 30, None) == \
        kiln_amd.KILN_EUNSUPPORTED
    assert L.kiln_dit_self_attn_x16(q, 1, 512, q, q, q, q, 1e-6, q, q, 5, 96, 4, q, 1 << 30, None) == \
        kiln_amd.KILN_EUNSUPPORTED
    assert L.kiln_dit_self_attn_x16(q, 1, 512, q, q, q, q, 1e-6, q, q, 2, 96, 4, q, 16, None) == kiln_amd.KILN_ENOMEM
    assert L.kiln_dit_self_attn_x16(q, 1, 512, q, q, None, q, 1e-6, q, q, 2, 96, 4, q, 1 << 30, None) == \
        kiln_amd.KILN_EINVAL
    assert L.kiln_dit_self_attn_x16_workspace_bytes(0, 96, 4) == 0
    assert L.kiln_dit_cross_attn_x16(q, None, 1, 512, q, q, q, 1e-6, 2, 96, 4, q, q, q, None, 0, 0, 5.0, 2.5, 0.25,
                                     q, 16, None) == kiln_amd.KILN_ENOMEM
    # small passes and sampler steps: null pointers and sizes
    assert L.kiln_matvec_bf16(None, q, q, None, 4, 8, None) == kiln_amd.KILN_EINVAL
    assert L.kiln_matvec_bf16_grouped(q, q, q, None, -1, 4, 8, None) == kiln_amd.KILN_EINVAL
    assert L.kiln_patchify(q, q, 7, 8, None) == kiln_amd.KILN_EINVAL
    assert L.kiln_unpatchify(q, q, 32, 8, 8, None) == kiln_amd.KILN_EINVAL
    assert L.kiln_linear_f32(q, 4, q, 8, q, 3, 8, 8, None) == kiln_amd.KILN_EINVAL
    assert L.kiln_flow_euler_step(q, q, 0.0, 0.5, 16, None) == kiln_amd.KILN_EINVAL
    assert L.kiln_flow_update(None, q, None, 1.0, 0.0, 0.0, 16, None) == kiln_amd.KILN_EINVAL
    assert L.kiln_flow_inpaint_in(q, q, q, None, q, 0.5, 16, None) == kiln_amd.KILN_EINVAL
    assert L.kiln_rel_l1(q, q, 16, None, None) == kiln_amd.KILN_EINVAL
    assert L.kiln_torch_randn(None, 0, 32) == kiln_amd.KILN_EINVAL
    # more batch items than one launch takes
    assert L.kiln_dit_self_attn_fused(p, 1, 2048, p, p, p, 1, 2048, None, None, 1e-6, None, None, 5, 64, 16, None, 0,
                                      None) != kiln_amd.KILN_OK


def test_python_wrappers_raise_kiln_error(L):
    with pytest.raises(kiln_amd.KilnError) as e:
        kiln_amd._check(kiln_amd.KILN_EUNSUPPORTED)
    assert e.value.status == kiln_amd.KILN_EUNSUPPORTED


def test_cpp_host_header_compiles():
    """kiln_amd/host/kiln_gpu.hpp (the reference-named C++ mirror) compiles against the C ABI header."""
    import subprocess
    src = '#include "kiln_amd/host/kiln_gpu.hpp"\nint main() { kiln::set_stream(nullptr); return 0; }\n'
    r = subprocess.run(["/opt/rocm/bin/hipcc", "-std=c++17", "-fsyntax-only", "-x", "hip", "-", "-I", kiln_amd.os.path.dirname(kiln_amd._HERE)],
                       input=src, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


@pytest.mark.parametrize("seed", [0, 42, 123456789])
def test_torch_randn_host_matches_torch_fixture(seed):
    """kiln_torch_randn (the library's host torch_randn, engine/src/pipeline.cu:17-64) against the torch.randn bit
    patterns committed in tests/golden (torch's vectorized log/cos differ from libm by a few ulp)."""
    import json
    import os
    with open(os.path.join(os.path.dirname(__file__), "golden", f"randn_seed{seed}.json")) as f:
        fx = json.load(f)
    ref = np.array([int(b, 16) for b in fx["bits"]], dtype=np.uint32).view(np.float32)
    got = kiln_amd.torch_randn(seed, len(ref)).numpy()
    ulp = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert ulp.max() <= 4 and (ulp == 0).mean() > 0.7
