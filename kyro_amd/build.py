"""Builds libkyro_verify.so and libkyro_verify.a in-tree with hipcc for gfx950.

Run as ``python -m kyro_amd.build``. Objects go to ``kyro_amd/_build`` and compile in parallel;
both libraries land next to this file so the Python binding (and a GPU box that receives this
tree) finds them without installation. The static archive is what a Rust ``build.rs`` links
(``rustc-link-lib=static=kyro_verify``): each object carries its gfx950 code object and registers
it at program start, so a consumer links it with its own toolchain plus ``-lamdhip64 -lstdc++``.
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJDIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libkyro_verify.so")
STATIC_LIB = os.path.join(HERE, "libkyro_verify.a")
SOURCES = ["runtime.cpp", "upload.hip", "blocks_abi.cpp", "block_manager.cpp", "sample_abi.cpp", "ngram_abi.cpp",
           "paged_attention.hip", "paged_attention_hd.hip", "paged_attention_hd_wide.hip", "spec_verify.hip", "kv_append.hip", "sample.hip", "ngram.hip", "noalloc.hip"]
ARCH = "gfx950"
# Per-source flags. paged_attention.hip (the head-dim-128 MFMA kernels, bf16 and f32) takes MFMA
# results in VGPRs: by default the compiler kept the attention accumulators in AGPRs and copied
# them to VGPRs in every loop iteration (64 v_accvgpr_read per block pair in the two-tile
# kernel). In VGPR form those copies go, the kernels need 70-100 fewer registers and the
# four-tile kernel no longer spills: skewed prefix 151.0 -> 148.0 us, mixed GQA 64/8 396.3 ->
# 388.0 us, Llama-3-8B attention 167.8 -> 166.7 us. The other head dims' kernels keep the
# default (head dim 160 measured 271.7 -> 298.2 us and 256 432.5 -> 445.7 us in VGPR form).
EXTRA_FLAGS = {"paged_attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"]}

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # Keep the compiler from forming packed-fp32 VALU ops (v_pk_fma_f32 and friends).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
    "-Wall", "-Wno-unused-command-line-argument",
]


def _compile(src: str, objdir: str = OBJDIR, defines=()) -> str:
    obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, *EXTRA_FLAGS.get(src, []), *[f"-D{d}" for d in defines], "-c",
           os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".hip"):
        cmd[1:1] = ["-x", "hip"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False, defines=(), out: str = LIB) -> str:
    """Compiles every HIP/C++ source and links the shared library. Returns its path.
    ``defines`` (NAME=VALUE strings) and ``out`` build a tuning variant elsewhere."""
    objdir = OBJDIR if out == LIB else os.path.splitext(out)[0] + "_obj"
    os.makedirs(objdir, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
        objs = list(pool.map(lambda s: _compile(s, objdir, defines), SOURCES))
    tmp = out + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    archive = os.path.splitext(out)[0] + ".a"
    tmp_a = archive + ".tmp"
    if os.path.exists(tmp_a):
        os.remove(tmp_a)
    res = subprocess.run(["ar", "rcs", tmp_a, *objs], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"ar failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp_a, archive)
    if verbose:
        print(f"built {out} and {archive}")
    return out


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
