"""The C ABI from plain C: tests/c_abi/verify_step.c includes only include/*.h, links only
libkyro_verify.so, and runs a verify step (attention, greedy verification, n-gram drafts into
verification, the device error path). Compiled without a GPU; run on one."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "c_abi", "verify_step.c")
LIBDIR = os.path.join(ROOT, "kyro_amd")


def build(tmp_dir):
    exe = os.path.join(tmp_dir, "verify_step")
    cmd = ["gcc", "-std=c99", "-O2", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), SRC,
           "-L", LIBDIR, "-lkyro_verify", f"-Wl,-rpath,{LIBDIR}", "-lm", "-o", exe]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    return exe


def test_c_consumer_compiles(tmp_path):
    build(str(tmp_path))


@pytest.mark.gpu
def test_c_consumer_runs_a_verify_step(tmp_path, gpu):
    exe = build(str(tmp_path))
    res = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.strip() == "ok"
