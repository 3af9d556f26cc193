"""Host check of the bf16 stencil's 3x3-kernel operand construction (CPU only).

``tests/stencil_band_check.cpp`` builds every lane's Kmat^T operand the way the
kernel does (``slime_amd/csrc/stencil_band.hpp``: a band-table run and v_perm_b32 byte
selectors) and compares it with the dense band matrix of the reference's 3x3
neighbourhood (weights ``slime/core/pseudopod.cu:151-154``, taps ``:170-179``; toroidal
here, decision D2): every element of every lane, for
four sets of weights. A planted mistake (the table's A and B words exchanged) is
reported.
"""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "stencil_band_check.cpp")


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("band") / "stencil_band_check")
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Werror", "-o", exe, SRC], check=True)
    return exe


def test_band_operands_equal_the_dense_kernel_matrix(checker):
    r = subprocess.run([checker], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and r.stdout.startswith("OK"), r.stdout
    assert "2048 operand elements" in r.stdout or int(r.stdout.split()[1]) == 4 * 32 * 4 * 2 * 8


def test_band_check_reports_a_planted_mistake(checker):
    r = subprocess.run([checker, "swap-ab"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "FAIL" in r.stdout, r.stdout
