"""CPU: the C ABI's host code under AddressSanitizer and
UndefinedBehaviorSanitizer (tests/sanitize/): descriptor validation,
workspace sizing over ~117 000 descriptors (every kernel family's sizing),
batch sizing and the argument checks that return before any launch.  The
library sources are built with the sanitizers on the host code only
(``-Xarch_host -fsanitize=...``); the driver launches no kernel, so it runs
without a GPU."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sanitize")


@pytest.mark.skipif(shutil.which("make") is None or not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="needs make and hipcc")
def test_capi_host_code_clean_under_asan_ubsan():
    build = subprocess.run(["make", "-C", HERE, "-j8"], capture_output=True, text=True)
    assert build.returncode == 0, build.stdout[-2000:] + build.stderr[-2000:]
    # the ASan runtime is linked into the executable; other preloaded
    # libraries of the environment may precede it in the load order
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    run = subprocess.run([os.path.join(HERE, "_build", "capi_sanitize")], capture_output=True, text=True,
                         env=env, timeout=300)
    out = run.stdout + run.stderr
    assert run.returncode == 0, out[-4000:]
    assert "ok: 0 failures" in out
    assert "runtime error" not in out and "AddressSanitizer" not in out
