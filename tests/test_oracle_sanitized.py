"""The oracle's CPU tests once more against a build of the restatement under
AddressSanitizer and UndefinedBehaviorSanitizer (host code only; the
reference runs its x86 kernels the same way, src/kernels/x86/kernels32.c:
101-109).  The sanitized library (oracle/_san/liboracle.so, `make -C oracle
sanitize`) is loaded in a child interpreter with the ASan runtime preloaded;
any finding aborts the child, so this test fails."""
import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _runtime(name):
    cc = shutil.which("gcc")
    if cc is None:
        return None
    p = subprocess.run([cc, f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    return p if os.path.isabs(p) and os.path.exists(p) else None


@pytest.mark.timeout(600)
def test_oracle_tests_clean_under_asan_ubsan():
    asan = _runtime("libasan.so")
    if asan is None or _runtime("libubsan.so") is None:
        pytest.skip("gcc sanitizer runtimes not installed")
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "sanitize"], check=True)
    lib = ROOT / "oracle" / "_san" / "liboracle.so"
    probe = "import pyoracle; print(pyoracle.ORACLE_SO)"
    env = dict(os.environ, LD_PRELOAD=asan, QWEN35_ORACLE_SO=str(lib),
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1",
               PYTHONPATH=os.pathsep.join([str(ROOT / "oracle"), str(ROOT)]))
    got = subprocess.run([sys.executable, "-c", probe], env=env, capture_output=True, text=True, check=True)
    assert got.stdout.strip() == str(lib)
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                        "tests/test_oracle_pins.py", "tests/test_synth.py"],
                       cwd=ROOT, env=env, capture_output=True, text=True)
    tail = (r.stdout + r.stderr)[-3000:]
    assert r.returncode == 0, tail
    assert "AddressSanitizer" not in tail and "runtime error" not in tail, tail
    assert " passed" in tail and "failed" not in tail, tail
