"""Host code under AddressSanitizer and UBSan (CPU, no GPU).

The library's host C++ (ABI runtime and argument checks, block manager and radix cache, n-gram
table, balanced-schedule plan query) and the oracle are built with -fsanitize=address,undefined
(tests/sanitize/build_sanitized.py), and the host-logic tests run against those builds in a
subprocess: the block-manager reference and random-stream tests, the n-gram tests, the plan
tests, the ABI argument checks and every oracle test. Any sanitizer report fails the run.
"""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST_TESTS = ["tests/test_block_manager.py", "tests/test_ngram.py", "tests/test_attention_plan.py", "tests/test_abi.py",
              "tests/test_oracle.py", "tests/test_golden.py", "tests/test_kv_append_oracle.py",
              "tests/test_sample_oracle.py"]


def _sanitized(tmp_path):
    from tests.sanitize import build_sanitized as bs

    lib, f64, f32 = bs.build(str(tmp_path))
    return bs, (lib, f64, f32), bs.environment(lib, f64, f32)


def test_host_code_under_sanitizers(tmp_path):
    bs, libs, env = _sanitized(tmp_path)
    # the sanitized builds are the ones the bindings load
    probe = ("import kyro_amd, oracle; kyro_amd.lib(); oracle._lib('f64'); oracle._lib('f32');"
             "print(open('/proc/self/maps').read())")
    maps = subprocess.run([sys.executable, "-c", probe], cwd=ROOT, env=env, capture_output=True, text=True,
                          timeout=300)
    assert maps.returncode == 0, maps.stderr[-3000:]
    for path in libs:
        assert path in maps.stdout, path
    res = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-m", "not gpu", "-p", "no:cacheprovider",
                          *HOST_TESTS], cwd=ROOT, env=env, capture_output=True, text=True, timeout=1200)
    out = res.stdout + res.stderr
    assert res.returncode == 0, out[-4000:]
    assert "AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
    assert " passed" in res.stdout


def test_sanitizers_are_live(tmp_path):
    """The flags and runtimes the run above uses do report: a planted heap overflow and a planted
    signed overflow each end the program with a sanitizer report."""
    from tests.sanitize import build_sanitized as bs

    src = tmp_path / "planted.c"
    src.write_text(
        "#include <limits.h>\n#include <stdlib.h>\n"
        "int main(int argc, char** argv) {\n"
        "  if (argv[1][0] == 'a') { int* p = malloc(4 * sizeof(int)); p[argc + 2] = 1; free(p); }\n"
        "  else { int x = INT_MAX - 1 + argc; return x + atoi(argv[1] + 1); }\n"
        "  return 0;\n}\n")
    exe = str(tmp_path / "planted")
    subprocess.run(["gcc", *bs.SANITIZE, "-o", exe, str(src)], check=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0", UBSAN_OPTIONS="print_stacktrace=1")
    heap = subprocess.run([exe, "a"], env=env, capture_output=True, text=True)
    # UBSan's object-size check or ASan's shadow check, whichever fires first
    assert heap.returncode != 0 and ("heap-buffer-overflow" in heap.stderr or "insufficient space" in heap.stderr)
    ub = subprocess.run([exe, "u5"], env=env, capture_output=True, text=True)
    assert ub.returncode != 0 and "signed integer overflow" in ub.stderr
