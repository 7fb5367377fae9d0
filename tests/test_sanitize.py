"""The host code under AddressSanitizer and UndefinedBehaviorSanitizer (the reference builds with API and shader
validation on, metal/CMakeLists.txt:71-72; its host-side analogue here is the sanitizers).

stratametal_amd/lib/libsmoe_asan.so is the library with its host code (the C ABI's checks and launches, the GGUF
reader, which parses untrusted files) built with -fsanitize=address,undefined (stratametal_amd/build.py
build_sanitized); oracle/_asan/liboracle.so is the CPU checker built the same way (oracle/Makefile, target asan).
The CPU tests that drive that code -- the GGUF reader's parsing and refusals, the C ABI's refusals, the oracle
against its pins -- run in a child process on both libraries, under the clang sanitizer runtime, and must pass with
no sanitizer report (any report aborts the child: halt_on_error, no recovery from undefined behaviour).
"""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "stratametal_amd", "lib", "libsmoe_asan.so")
ORACLE = os.path.join(ROOT, "oracle", "_asan", "liboracle.so")
CLANG = "/opt/rocm/llvm/bin/clang"
SUITES = ["tests/test_gguf.py", "tests/test_abi.py", "tests/test_oracle.py", "tests/test_oracle_native.py",
          "tests/test_oracle_hc.py", "tests/test_oracle_cache.py", "tests/test_stagewise.py"]


def _runtime():
    if not os.path.exists(CLANG):
        return None
    out = subprocess.run([CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    path = out.stdout.strip()
    return path if out.returncode == 0 and os.path.isabs(path) and os.path.exists(path) else None


@pytest.fixture(scope="module")
def env():
    rt = _runtime()
    if rt is None:
        pytest.skip("no clang sanitizer runtime in this image")
    if not os.path.exists(ORACLE):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "asan"], check=True)
    if not os.path.exists(LIB):
        kernels = os.path.join(ROOT, "stratametal_amd", "_build", "smoe_decode.o")
        if not os.path.exists(kernels):
            pytest.skip("the kernel objects are not built (python -m stratametal_amd.build)")
        sys.path.insert(0, ROOT)
        from stratametal_amd import build as B
        B.build_sanitized()
    e = dict(os.environ)
    e.update(LD_PRELOAD=rt, SMOE_LIB=LIB, SMOE_ORACLE_LIB=ORACLE,
             ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
             UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    return e


def test_sanitized_libraries_are_the_ones_loaded(env):
    code = ("import stratametal_amd as S, oracle as O; S.lib(); O.lib(); "
            "print(open('/proc/self/maps').read())")
    out = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr[-3000:]
    maps = out.stdout
    assert "libsmoe_asan.so" in maps and "/_asan/liboracle.so" in maps and "libclang_rt.asan" in maps
    assert "/lib/libsmoe.so" not in maps


def test_cpu_suites_under_sanitizers(env):
    cmd = [sys.executable, "-m", "pytest", *SUITES, "-m", "not gpu", "-q", "-x", "-p", "no:cacheprovider"]
    out = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    text = out.stdout + out.stderr
    assert "ERROR: AddressSanitizer" not in text, text[-4000:]
    assert "runtime error:" not in text, text[-4000:]
    assert out.returncode == 0, text[-4000:]
    assert " passed" in out.stdout
