"""Host code under AddressSanitizer + UndefinedBehaviorSanitizer (CPU only).
The library: the GGUF and .qmoe parsers fed well-formed, split, truncated and
damaged files, and the C-ABI's host-side argument checks, through a build of
the same sources with the host side sanitized (`make -C fomoe_amd
host-sanitize`) loaded in place of the product library by a child pytest run
with clang's ASan runtime preloaded. The oracle's C restatement likewise
(`make -C oracle sanitize`, gcc's runtime, its own child run). Any report
fails the run."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN_LIB = os.path.join(ROOT, "fomoe_amd", "_build_san", "libfomoe_host_san.so")
CLANG = "/opt/rocm/llvm/bin/clang"

# host-only tests of the library (the gfx950 check reads the product binary,
# and the link test builds against the product library by name)
SELECTION = ["tests/test_gguf.py", "tests/test_qmoe.py", "tests/test_abi.py"]
DESELECT = "not gfx950_only and not translation_unit"


def _asan_runtime():
    r = subprocess.run([CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    path = r.stdout.strip()
    return path if r.returncode == 0 and os.path.isabs(path) and os.path.exists(path) else None


@pytest.mark.skipif(shutil.which("make") is None or not os.path.exists(CLANG), reason="no hipcc toolchain")
def test_host_code_under_asan_and_ubsan():
    rt = _asan_runtime()
    if rt is None:
        pytest.skip("clang ASan runtime not found")
    r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "fomoe_amd"), "-j8", "host-sanitize"],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    env = dict(os.environ, FOMOE_LIB=SAN_LIB, LD_PRELOAD=rt,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0:exitcode=99",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1:exitcode=98")
    cmd = [sys.executable, "-m", "pytest", "-q", "-x", "-m", "not gpu", "-p", "no:cacheprovider",
           "-k", DESELECT] + SELECTION
    r = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    out = r.stdout[-4000:] + r.stderr[-4000:]
    assert r.returncode == 0, out
    assert "ERROR: AddressSanitizer" not in out and "runtime error:" not in out, out
    assert " passed" in r.stdout, out


def _gcc_asan():
    r = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True)
    path = os.path.realpath(r.stdout.strip()) if r.returncode == 0 else ""
    return path if os.path.isabs(path) and os.path.exists(path) else None


@pytest.mark.skipif(shutil.which("make") is None or shutil.which("gcc") is None, reason="no gcc")
def test_oracle_under_asan_and_ubsan():
    rt = _gcc_asan()
    if rt is None:
        pytest.skip("gcc ASan runtime not found")
    r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "sanitize"],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    env = dict(os.environ, ORACLE_LIB=os.path.join(ROOT, "oracle", "_san", "liboracle_san.so"), LD_PRELOAD=rt,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:exitcode=99",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1:exitcode=98")
    cmd = [sys.executable, "-m", "pytest", "-q", "-x", "-m", "not gpu", "-p", "no:cacheprovider",
           "tests/test_oracle.py"]
    r = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    out = r.stdout[-4000:] + r.stderr[-4000:]
    assert r.returncode == 0, out
    assert "ERROR: AddressSanitizer" not in out and "runtime error:" not in out, out
    assert " passed" in r.stdout, out
