"""The C ABI's host-side argument validation under AddressSanitizer and
UndefinedBehaviorSanitizer, without a GPU: tests/test_abi.py runs in a child
python against ``pare_amd.build.build_sanitized()``'s library (capi.hip with
ASan and UBSan in the host pass), with the clang ASan runtime preloaded.
Any sanitizer report fails the child (halt_on_error; UBSan does not recover)."""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_abi_validation_clean_under_asan_and_ubsan():
    from pare_amd.build import asan_runtime, build_sanitized

    lib = build_sanitized()
    # the library really is instrumented (ASan and UBSan entry points)
    syms = subprocess.run(["nm", "-D", str(lib)], capture_output=True, text=True).stdout
    assert "__asan_" in syms and "__ubsan_" in syms
    env = dict(os.environ)
    env["LD_PRELOAD"] = str(asan_runtime())
    # python itself is not instrumented: its allocations at exit are not ours
    env["ASAN_OPTIONS"] = "detect_leaks=0:halt_on_error=1:abort_on_error=0"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    boot = ("import sys; sys.path.insert(0, %r); import pare_amd._lib as L; "
            "from pathlib import Path; L.LIB_PATH = Path(%r); import pytest; "
            "sys.exit(pytest.main(['-q', '-p', 'no:cacheprovider', %r]))"
            % (str(ROOT), str(lib), str(ROOT / "tests" / "test_abi.py")))
    res = subprocess.run([sys.executable, "-c", boot], cwd=ROOT, env=env, capture_output=True,
                         text=True, timeout=600)
    out = res.stdout + res.stderr
    print(out[-3000:])
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-3000:]
    assert res.returncode == 0, out[-3000:]
    # the child ran the sanitized library, not the package's own build
    assert "passed" in res.stdout
