"""include/aq.h from compiled C: tests/c/aq_capi_check.c (built with gcc by
tests/c/Makefile, from __graft_entry__.build()) uploads Q4_K, Q6_K and Q8_0
weights through the C ABI, runs aq_qmatmul_f32 at m = 1, 3 and 40, and
checks the outputs (1e-5), the integer block sums (bit-exact) and the
quantised activations (byte-exact) against the C oracle, plus the error
statuses for a wrong k, a null pointer and a short byte count.  It runs as a
child process, as the Rust NIF would call the library from its own process."""
import os
import subprocess

import pytest

import arm_ai_amd as A

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "c", "build", "aq_capi_check")


def _run():
    if not os.path.exists(EXE):
        pytest.fail(f"{EXE} is not built: run __graft_entry__.build() (make -C tests/c)")
    return subprocess.run([EXE], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=300)


@pytest.mark.skipif(A.device_count() > 0, reason="checks the no-device path")
def test_c_program_links_and_reports_no_device():
    r = _run()
    assert "aq_abi_version 1" in r.stdout
    assert r.returncode == 1 and "no device" in r.stdout


@pytest.mark.gpu
def test_c_program_against_the_oracle():
    r = _run()
    print(r.stdout)
    assert r.returncode == 0, r.stdout[-3000:]
    assert r.stdout.rstrip().endswith("ALL OK")
    assert r.stdout.count("bit-exact") == 9  # three weight types x three batch sizes
