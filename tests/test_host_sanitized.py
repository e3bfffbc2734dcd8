"""The host library (page allocator, refcounts, radix tree, block manager)
rebuilt with AddressSanitizer and UndefinedBehaviorSanitizer, and the host
tests run against that build in a child process: an out-of-bounds access, a
use after free or undefined behaviour in kv_host.cpp aborts the child and
fails this test. The product library is left untouched. CPU only."""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

from mitten_amd import _build

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST_TESTS = ["tests/test_host_kv.py", "tests/test_workloads.py"]


def _runtime(name: str) -> str | None:
    cxx = os.environ.get("CXX", "g++")
    try:
        out = subprocess.run([cxx, f"-print-file-name={name}"], capture_output=True, text=True, check=True)
    except (OSError, subprocess.CalledProcessError):
        return None
    path = out.stdout.strip()
    return path if os.path.isabs(path) and os.path.exists(path) else None


def test_host_library_under_address_and_undefined_behaviour_sanitizers(tmp_path):
    asan, ubsan = _runtime("libasan.so"), _runtime("libubsan.so")
    if not (asan and ubsan):
        pytest.skip("the compiler's sanitizer runtimes are not installed")
    lib = str(tmp_path / "libmitten_kvhost_sanitized.so")
    sanitize = ["-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
                "-fno-sanitize-recover=undefined"]
    build = subprocess.run(_build.host_cmd(lib, sanitize), capture_output=True, text=True)
    assert build.returncode == 0, build.stderr[-4000:]
    # The child points the loader at the sanitized build before the first
    # host call, then runs the host tests without output capture, so that a
    # sanitizer report (written to stderr just before the child exits)
    # reaches this test's failure message. The wall-clock bound on the
    # scheduler's overhead is left out: it measures the plain build (the
    # plain CPU suite runs it), and the sanitizers' instrumentation slows the
    # calls it times.
    child = (
        "import sys; sys.path.insert(0, {root!r}); from mitten_amd import _build; "
        "_build.HOST_LIB = {lib!r}; import pytest; "
        "sys.exit(pytest.main(['-q', '-s', '-x', '-p', 'no:cacheprovider', '-m', 'not gpu', "
        "'-k', 'not scheduler_overhead_bound'] + {tests!r}))"
    ).format(root=ROOT, lib=lib, tests=[os.path.join(ROOT, t) for t in HOST_TESTS])
    env = dict(os.environ, LD_PRELOAD=f"{asan}:{ubsan}", ASAN_OPTIONS="detect_leaks=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    run = subprocess.run([sys.executable, "-c", child], cwd=ROOT, env=env, capture_output=True, text=True,
                         timeout=900)
    assert run.returncode == 0, run.stdout[-4000:] + run.stderr[-4000:]
    assert " passed" in run.stdout
