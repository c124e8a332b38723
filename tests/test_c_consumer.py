"""The C ABI from plain C: tests/c_abi/verify_step.c includes only include/*.h and runs a verify
step (attention, greedy verification, n-gram drafts into verification, the device error path).

It is linked two ways with plain gcc, no hipcc: against libkyro_verify.so, and against the static
archive libkyro_verify.a plus the ROCm runtime (-lamdhip64 -lstdc++), which is how a Rust build.rs
links the library (rustc-link-lib=static=kyro_verify). Compiled without a GPU; run on one."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "c_abi", "verify_step.c")
LIBDIR = os.path.join(ROOT, "kyro_amd")
ROCM_LIB = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib")


def build(tmp_dir, link):
    exe = os.path.join(tmp_dir, f"verify_step_{link}")
    cmd = ["gcc", "-std=c99", "-O2", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), SRC]
    if link == "shared":
        cmd += ["-L", LIBDIR, "-lkyro_verify", f"-Wl,-rpath,{LIBDIR}"]
    else:
        # rustc links executables with --gc-sections and --as-needed: the objects' code-object
        # registration (constructors in .init_array) must survive both.
        cmd += ["-Wl,--gc-sections", "-Wl,--as-needed", os.path.join(LIBDIR, "libkyro_verify.a"), "-L", ROCM_LIB,
                "-lamdhip64", "-lstdc++", f"-Wl,-rpath,{ROCM_LIB}"]
    cmd += ["-lm", "-o", exe]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    return exe


@pytest.mark.parametrize("link", ["shared", "static"])
def test_c_consumer_compiles(tmp_path, link):
    exe = build(str(tmp_path), link)
    if link == "static":  # the archive's code is in the executable, not loaded from the .so
        deps = subprocess.run(["ldd", exe], capture_output=True, text=True).stdout
        assert "libkyro_verify" not in deps and "libamdhip64" in deps


@pytest.mark.gpu
@pytest.mark.parametrize("link", ["shared", "static"])
def test_c_consumer_runs_a_verify_step(tmp_path, gpu, link):
    exe = build(str(tmp_path), link)
    res = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.strip() == "ok"
