"""The C-ABI tests again under host AddressSanitizer.

``myvllm_amd.build.build_asan()`` compiles gdn_capi.cpp (argument validation,
descriptor decoding, error mapping) with ``-fsanitize=address`` on the host
side only and links it with the kernels' objects of the last build; a fresh
interpreter loads that library through MYVLLM_AMD_LIB with the sanitizer
runtime preloaded and runs tests/test_capi.py.  Any invalid read or write the
validation layer makes on a descriptor turns into an AddressSanitizer report
and a failing run.  CPU only.
"""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _asan_env():
    from myvllm_amd import build as B

    missing = [s for s in B.SOURCES if s != "gdn_capi.cpp"
               and not os.path.exists(os.path.join(B.OBJDIR, os.path.splitext(s)[0] + ".o"))]
    if missing:
        pytest.skip(f"kernel objects not built ({missing[0]}): run the normal build first")
    lib = B.build_asan()
    env = dict(os.environ, MYVLLM_AMD_LIB=lib, LD_PRELOAD=B.asan_runtime(),
               ASAN_OPTIONS="detect_leaks=0:exitcode=23")
    return lib, env


def test_capi_under_address_sanitizer():
    lib, env = _asan_env()
    probe = subprocess.run(
        [sys.executable, "-c",
         "from myvllm_amd import _lib; _lib.load(); import ctypes;"
         "print(_lib.LIB_PATH, hasattr(ctypes.CDLL(_lib.LIB_PATH), '__asan_report_load4'))"],
        cwd=ROOT, env=env, capture_output=True, text=True, timeout=300)
    assert probe.returncode == 0, probe.stdout + probe.stderr
    assert probe.stdout.split() == [lib, "True"], probe.stdout
    res = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", "tests/test_capi.py"],
                         cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    out = res.stdout + res.stderr
    assert "AddressSanitizer" not in out, out[-4000:]
    assert res.returncode == 0, out[-4000:]
