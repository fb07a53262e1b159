"""The C++ harnesses (built by tests/cpp/build.sh): tests/cpp/attn_test (the reference's bench/tfa_test.cu shapes
and inputs) and tests/cpp/dit_section_test (the DiT block attention section with contexts, padding and NAG),
both through the C++ host mirror kiln_amd/host/kiln_gpu.hpp and the C ABI."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def test_cpp_attn_harness(gpu):
    exe = os.path.join(HERE, "cpp", "attn_test")
    src = os.path.join(HERE, "cpp", "attn_test.cpp")
    if not os.path.exists(exe) or os.path.getmtime(exe) < os.path.getmtime(src):
        subprocess.run(["bash", os.path.join(HERE, "cpp", "build.sh")], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=100)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr


def test_cpp_dit_section(gpu):
    exe = os.path.join(HERE, "cpp", "dit_section_test")
    src = os.path.join(HERE, "cpp", "dit_section_test.cpp")
    if not os.path.exists(exe) or os.path.getmtime(exe) < os.path.getmtime(src):
        subprocess.run(["bash", os.path.join(HERE, "cpp", "build.sh")], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=100)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
