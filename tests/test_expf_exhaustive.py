"""The device exp (uq_expf in uefi-gpu_amd/csrc/uq_device.h) against the
oracle's libm-0.2.16 expf (uqo_expf; driver/src/frontier_cpu_expf.rs:80-170)
on every f32 input.

uq_expf is branch-free: the argument reduction's cases, the small-|x| result,
the special values and scalbnf's pre-scaling are selects. The check builds
that same header function for the host (hipcc, host pass only, no contraction)
and compares all 2^32 inputs bit for bit, so a changed constant, case
boundary or scaling step that alters any result fails here. The GPU build of
the same source is covered by the softmax, SiLU and attention parity tests.
"""
import os
import shutil
import subprocess

import pytest

import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_device_expf_source_matches_oracle_on_all_inputs(tmp_path):
    O.lib()  # the oracle library is built and loadable
    exe = str(tmp_path / "expf_check")
    oracle_dir = os.path.dirname(O.LIB_PATH)
    subprocess.run([HIPCC, "-x", "hip", "--cuda-host-only", "-O2", "-ffp-contract=off", "-std=c++17", "-o", exe,
                    os.path.join(ROOT, "tests", "expf_exhaustive.cpp"), "-L", oracle_dir, "-loracle",
                    "-Wl,-rpath," + oracle_dir, "-pthread"], check=True, capture_output=True)
    threads = str(min(8, os.cpu_count() or 1))
    r = subprocess.run([exe, threads], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout
    assert "inputs differing: 0 of 2^32" in r.stdout
