"""The host side of the library (w64_host.cpp: table build, both encoders,
the host decoder) built with g++ under AddressSanitizer and
UndefinedBehaviorSanitizer, and driven through tests/host_sanitizer_driver.py
in a child process with the sanitizer runtime preloaded: no report on
valid, rejected or corrupted inputs."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_host_code_under_asan_ubsan(tmp_path):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    asan = subprocess.run(["g++", "-print-file-name=libasan.so"], capture_output=True,
                          text=True).stdout.strip()
    if not os.path.isabs(asan) or not os.path.exists(asan):
        pytest.skip("no AddressSanitizer runtime")
    so = str(tmp_path / "libhost_asan.so")
    subprocess.check_call(
        ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
         "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer", "-shared", "-fPIC",
         "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", "-o", so,
         os.path.join(ROOT, "vram-compression_amd", "csrc", "w64_host.cpp"), "-lpthread"],
        stderr=subprocess.DEVNULL)
    env = dict(os.environ, LD_PRELOAD=asan, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([sys.executable, os.path.join(ROOT, "tests", "host_sanitizer_driver.py"), so],
                       capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert r.stdout.strip().startswith("ok "), r.stdout[-2000:]
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr[-4000:]
