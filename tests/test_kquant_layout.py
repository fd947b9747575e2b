"""The K-quant layout code of the device header (uefi-gpu_amd/csrc/uq_units.h:
Q3K::pack_unit, unit_parts and words, the row-block Q3KSB::pack/unpack and
sb_geom/sb_piece, the source of the upload repacks, their
verify kernels and the matvecs' bit assembly) built for the host and checked
against the oracle (uqo_q3k_block_dots, uqo_matvec_x; oracle/uq_oracle.c, whose
Q3_K decode follows ggml's dequantize_row_q3_K and is pinned by the byte-literal
known-answer blocks of test_oracle_core.py) on seeded GGUF rows of 1 to 8
superblocks: every value's bits round-trip, every 16-value integer dot matches,
and every row sum is within 1 ulp. The GPU build of the same source is covered
by the Q3_K matvec, gate/up and MoE parity tests.
"""
import os
import shutil
import subprocess

import pytest

import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_q3k_unit_layout_matches_oracle(tmp_path):
    O.lib()  # the oracle library is built and loadable
    exe = str(tmp_path / "kquant_layout_check")
    oracle_dir = os.path.dirname(O.LIB_PATH)
    subprocess.run([HIPCC, "-x", "hip", "--cuda-host-only", "-O2", "-ffp-contract=off", "-std=c++17", "-o", exe,
                    os.path.join(ROOT, "tests", "kquant_layout_check.cpp"), "-L", oracle_dir, "-loracle",
                    "-Wl,-rpath," + oracle_dir, "-pthread"], check=True, capture_output=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout
    assert "parts differing: 0, dots differing: 0, rows beyond 1 ulp: 0 of 96" in r.stdout
    assert "row-block round trips differing: 0, geometry faults: 0" in r.stdout
