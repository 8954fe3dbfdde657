"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer.

The library is rebuilt with both sanitizers on its host code
(opaque_amd.build.build_sanitized; device code as usual) and the argument,
table and error-text checks of tests/test_abi.py run against it in a child
process that preloads the sanitizer runtime and stops at the first report.
No GPU is needed: every call returns before any device work.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

from opaque_amd import build

ROOT = Path(__file__).resolve().parents[1]


def test_abi_checks_are_clean_under_sanitizers():
    rt = build.sanitizer_runtime()
    if rt is None:
        pytest.skip("no AddressSanitizer runtime next to hipcc")
    lib = build.build_sanitized()
    env = dict(os.environ)
    env.update({
        "OPAQUE_AMD_LIBRARY": str(lib),
        "LD_PRELOAD": str(rt),
        # Python and torch keep memory until exit: leak reports are noise here.
        "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=0:halt_on_error=1:exitcode=86",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1:exitcode=87",
    })
    probe = subprocess.run([sys.executable, "-c", "from opaque_amd import _native as N; print(N.load()._name)"],
                           cwd=ROOT, env=env, capture_output=True, text=True, timeout=300)
    assert probe.returncode == 0 and probe.stdout.strip() == str(lib), probe.stdout + probe.stderr
    proc = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider",
                           str(ROOT / "tests" / "test_abi.py"), "-m", "not gpu"],
                          cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    out = proc.stdout[-3000:] + proc.stderr[-3000:]
    assert proc.returncode == 0, out
    assert "AddressSanitizer" not in out and "runtime error" not in out, out
    assert " passed" in proc.stdout, out
