"""Host-only sanitizer build for the CPU tests (no GPU code is instrumented).

The library's host C++ (ABI runtime, block manager and radix cache, n-gram table, sampler
arguments) is compiled with g++ under AddressSanitizer and UBSan and linked with the ordinary
kernel objects of the in-tree build; the oracle is compiled with gcc the same way. Loading them
needs gcc's sanitizer runtimes preloaded (``preload()``), since the Python interpreter is not
instrumented.
"""
from __future__ import annotations

import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
CSRC = os.path.join(ROOT, "kyro_amd", "csrc")
OBJDIR = os.path.join(ROOT, "kyro_amd", "_build")
ORACLE_SRC = os.path.join(ROOT, "oracle", "kyro_oracle.c")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HOST_SOURCES = ["runtime.cpp", "blocks_abi.cpp", "block_manager.cpp", "sample_abi.cpp", "ngram_abi.cpp"]
SANITIZE = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(" ".join(cmd) + "\n" + res.stdout + res.stderr)


def kernel_objects():
    """The in-tree build's objects of the .hip sources (kernels and their launchers)."""
    from kyro_amd import build as kb

    objs = [os.path.join(OBJDIR, os.path.splitext(s)[0] + ".o") for s in kb.SOURCES if s.endswith(".hip")]
    if not all(os.path.exists(o) for o in objs):
        kb.build()
    return objs


def build(outdir: str):
    """Returns (library, f64 oracle, f32 oracle) paths of the sanitized builds in ``outdir``."""
    import concurrent.futures

    os.makedirs(outdir, exist_ok=True)
    host = [os.path.join(outdir, os.path.splitext(src)[0] + ".o") for src in HOST_SOURCES]
    lib = os.path.join(outdir, "libkyro_verify_san.so")
    oracles = [os.path.join(outdir, "libkyro_oracle_san.so"), os.path.join(outdir, "libkyro_oracle_f32_san.so")]
    cmds = [["g++", "-std=c++17", "-fPIC", *SANITIZE, "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROCM, "include"),
             "-I", os.path.join(ROOT, "include"), "-I", CSRC, "-c", os.path.join(CSRC, src), "-o", obj]
            for src, obj in zip(HOST_SOURCES, host)]
    cmds += [["gcc", "-std=c11", "-fPIC", "-shared", *SANITIZE, *extra, "-o", out, ORACLE_SRC, "-lm", "-lpthread"]
             for out, extra in zip(oracles, ([], ["-DORACLE_F32"]))]
    kernels = kernel_objects()
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(cmds))) as pool:
        list(pool.map(_run, cmds))
    _run(["g++", "-shared", *SANITIZE, "-o", lib, *host, *kernels, "-L", os.path.join(ROCM, "lib"),
          "-lamdhip64", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}"])
    return lib, oracles[0], oracles[1]


def preload() -> str:
    """LD_PRELOAD value for gcc's AddressSanitizer and UBSan runtimes."""
    libs = []
    for name in ("libasan.so", "libubsan.so"):
        path = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
        libs.append(path)
    return ":".join(libs)


def environment(lib: str, f64: str, f32: str) -> dict:
    env = dict(os.environ)
    env.update(KYRO_VERIFY_LIB=lib, KYRO_ORACLE_LIB=f64, KYRO_ORACLE_F32_LIB=f32, LD_PRELOAD=preload(),
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    return env
