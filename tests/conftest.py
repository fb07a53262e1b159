import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


@pytest.fixture(scope="session")
def gpu():
    """The HIP library, loaded on a machine with a GPU. No fallback: missing library or GPU fails."""
    import torch
    import kiln_amd
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a GPU")
    L = kiln_amd.lib()
    buf = __import__("ctypes").create_string_buffer(64)
    assert L.kiln_attn_device_arch(0, buf, 64) == 0
    arch = buf.value.decode()
    assert arch.startswith("gfx950"), f"expected gfx950, found {arch}"
    return L
