"""The product range-coder core (csrc/rc_core.h, the code the kernels run) built for the CPU with g++ under
AddressSanitizer + UndefinedBehaviorSanitizer, and checked by tests/native/coder_host_check.cpp: the
division-free decoder target against exact u64 division (random, corrupt-stream and boundary states), the
encoder's words against the oracle coder, round trips, and overflow handling."""
import os
import shutil
import subprocess

import pytest

from conftest import PKG, REPO


@pytest.mark.skipif(shutil.which("g++") is None or shutil.which("gcc") is None, reason="needs gcc/g++")
def test_product_coder_on_cpu_under_sanitizers(tmp_path):
    san = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]
    obj = tmp_path / "rc_oracle.o"
    subprocess.run(["gcc", "-std=c11", "-O1", "-g", "-ffp-contract=off", *san, "-c",
                    os.path.join(REPO, "oracle", "rc_oracle.c"), "-o", str(obj)], check=True)
    exe = tmp_path / "coder_host_check"
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-Wall", "-Wextra", *san,
                    "-I", os.path.join(PKG, "csrc"), os.path.join(REPO, "tests", "native", "coder_host_check.cpp"),
                    str(obj), "-lm", "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300,
                       env={**os.environ, "ASAN_OPTIONS": "detect_leaks=1", "UBSAN_OPTIONS": "print_stacktrace=1"})
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "failures 0" in r.stdout
