"""The C ABI's host code (tda_amd/csrc/tda_host.cpp) built alone with g++ under
AddressSanitizer and UndefinedBehaviorSanitizer, with stub launchers in place of the kernels
(tests/sanitize/stub_launch.cpp), and driven through every validation path, the buffer sizes
and the parameter blocks handed to the launchers (tests/sanitize/abi_driver.cpp).  CPU only."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = os.path.join(ROOT, "tests", "sanitize")


def test_host_abi_under_asan_ubsan(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ missing")
    exe = tmp_path / "abi_driver"
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           os.path.join(ROOT, "tda_amd", "csrc", "tda_host.cpp"),
           os.path.join(SAN, "stub_launch.cpp"), os.path.join(SAN, "abi_driver.cpp"), "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    env.pop("LD_PRELOAD", None)
    r = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all checks passed" in r.stdout
