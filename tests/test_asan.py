"""The host library's C code (GGUF reader and writer, the C ABI's argument
checks) under AddressSanitizer: a g++ -fsanitize=address build of it runs
the CPU tests of the GGUF parser (including the truncated and malformed
files) and of the ABI in a child interpreter with the sanitizer's runtime
preloaded.  Any invalid read, write or double free aborts the child."""

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.timeout(900)
def test_gguf_and_abi_under_address_sanitizer():
    sys.path.insert(0, ROOT)
    from inferi_amd import build as B

    lib = B.build_host_asan()
    env = dict(os.environ)
    env.update(IFR_LIB=lib, LD_PRELOAD=B.asan_runtime(), ASAN_OPTIONS="detect_leaks=0:abort_on_error=1")
    probe = subprocess.run([sys.executable, "-c", "import inferi_amd as I; print(I.lib()._name)"], cwd=ROOT, env=env,
                           stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=300)
    assert probe.returncode == 0 and probe.stdout.strip().endswith("libinferi_hip_asan.so"), probe.stdout[-2000:]
    r = subprocess.run([sys.executable, "-m", "pytest", "tests/test_gguf.py", "tests/test_abi.py", "-q", "-m", "not gpu",
                        "-p", "no:cacheprovider"], cwd=ROOT, env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-4000:]
    assert "AddressSanitizer" not in r.stdout, r.stdout[-4000:]
