"""Host replay of the bf16 stencil's tile walk (CPU only).

``tests/stencil_sched_check.cpp`` runs the walk of ``slime_amd/csrc/stencil_sched.hpp``
(the functions the kernel calls) for every workgroup of a launch, with the ticket
draws and finish counts of all workgroups interleaved in seeded random orders, two
launches back to back on the same counters: every tile once per launch, each inside
its workgroup's XCD eighth, every counter zero after each launch. A planted mistake
(tickets starting one tile late) is reported.
"""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "stencil_sched_check.cpp")


def _build(tmp_path_factory, *defines):
    exe = str(tmp_path_factory.mktemp("sched") / "stencil_sched_check")
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Werror", *defines, "-o", exe, SRC], check=True)
    return exe


def test_every_tile_once_per_launch_and_counters_reset(tmp_path_factory):
    r = subprocess.run([_build(tmp_path_factory)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.startswith("OK"), r.stdout


def test_sched_check_reports_a_planted_mistake(tmp_path_factory):
    r = subprocess.run([_build(tmp_path_factory, "-DPLANT_FIRST")], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 1 and "processed 0 times" in r.stdout, r.stdout
