"""The oracle's tests again, against a build of the same C source under
AddressSanitizer and UndefinedBehaviorSanitizer (oracle/Makefile,
sanitize-test: gcc, host code only).  A memory error or undefined behaviour
in the restatement aborts the run."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_oracle_under_asan_ubsan():
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    asan = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    if not Path(asan).is_file():
        pytest.skip("gcc has no AddressSanitizer runtime here")
    r = subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "sanitize-test"], capture_output=True, text=True,
                       timeout=600)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    assert " passed" in r.stdout
