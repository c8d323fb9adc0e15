"""The CPU suite under AddressSanitizer + UBSan (tests/sanitize.sh): the C host layer
(platform, registry, operator host code, graph executor and fusion pass, session) and
the oracle, built with -fsanitize=address,undefined, must run every CPU test cleanly.
The reference gates its CUDA code on compute-sanitizer (scripts/run_sanitizer.sh:82-100);
here the device code runs only on the GPU box, so the gate is for host code."""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(os.environ.get("CUDAFORGE_SANITIZER_RUN") == "1", reason="already inside the sanitizer run")
@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc's sanitizer runtimes")
def test_cpu_suite_under_asan_and_ubsan():
    env = dict(os.environ, CUDAFORGE_SANITIZER_RUN="1")
    r = subprocess.run(["bash", os.path.join(ROOT, "tests", "sanitize.sh")], env=env, capture_output=True,
                       text=True, timeout=900)
    tail = (r.stdout + r.stderr)[-3000:]
    assert r.returncode == 0, tail
    assert " passed" in r.stdout and "ERROR: AddressSanitizer" not in tail and "runtime error" not in tail, tail
