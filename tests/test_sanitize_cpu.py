"""The CPU sanitizer run (tests/sanitize/run.sh): the oracle's C restatement
and the host GGUF reader built with AddressSanitizer + UndefinedBehavior-
Sanitizer; the oracle's CPU tests against the instrumented library, the GGUF
reader over well-formed, truncated and byte-flipped files.  Any test failure
or sanitizer report fails it."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None or shutil.which("g++") is None, reason="needs gcc / g++")
def test_sanitizer_run():
    r = subprocess.run(["bash", os.path.join(HERE, "sanitize", "run.sh")], capture_output=True, text=True,
                       timeout=600)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    assert "no sanitizer report" in r.stdout
