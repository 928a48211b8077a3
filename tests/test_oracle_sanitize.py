"""The CPU oracle built under AddressSanitizer and UndefinedBehaviorSanitizer
(oracle/Makefile `sanitize`): every oracle function runs once on small,
ragged inputs (oracle/sanitize_check.c) and any out-of-bounds access, leak or
undefined operation fails the run.  CPU only."""
import os
import shutil
import subprocess
from pathlib import Path

import pytest

ORACLE = Path(__file__).resolve().parents[1] / "oracle"


@pytest.mark.skipif(shutil.which("gcc") is None and shutil.which("cc") is None, reason="no C compiler")
def test_oracle_is_clean_under_asan_and_ubsan():
    subprocess.run(["make", "-s", "-C", str(ORACLE), "sanitize"], check=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:verify_asan_link_order=0", OMP_NUM_THREADS="2",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([str(ORACLE / "_san" / "sanitize_check")], capture_output=True, text=True,
                       env=env, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "sanitize_check: ok" in r.stdout
    assert "runtime error" not in r.stderr
