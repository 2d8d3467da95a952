"""The oracle under AddressSanitizer and UndefinedBehaviorSanitizer: the
sanitizer build of oracle/ (``make -C oracle asan``) runs the oracle's pin
tests and the C-ABI checks that use it, in a child process with the
sanitizer runtimes preloaded (the interpreter itself is not instrumented).
Any report stops that process with a non-zero status."""
import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _runtime(name):
    gcc = shutil.which("gcc")
    if not gcc:
        return None
    p = subprocess.run([gcc, f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    return p if p and os.path.isabs(p) and os.path.exists(p) else None


def test_oracle_tests_pass_under_asan_and_ubsan():
    asan, ubsan = _runtime("libasan.so"), _runtime("libubsan.so")
    if not (asan and ubsan):
        pytest.skip("gcc sanitizer runtimes not found")
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "asan"], check=True)
    lib = ROOT / "oracle" / "_asan" / "liboracle.so"
    syms = subprocess.run(["nm", "-D", str(lib)], capture_output=True, text=True).stdout
    assert "__asan" in syms and "__ubsan" in syms, "the oracle build is not instrumented"
    env = dict(os.environ, LD_PRELOAD=f"{asan}:{ubsan}", FMD_ORACLE_LIB=str(lib),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    code = ("import sys, pytest; from oracle import oracle; "
            f"assert str(oracle.LIB) == {str(lib)!r}; "
            "sys.exit(pytest.main(['-q', '-p', 'no:cacheprovider', '-m', 'not gpu', "
            "'tests/test_oracle.py', 'tests/test_oracle_encoder.py', 'tests/test_abi_cpu.py']))")
    proc = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True,
                          text=True, timeout=900)
    tail = (proc.stdout + proc.stderr)[-3000:]
    assert proc.returncode == 0, tail
    assert "ERROR: AddressSanitizer" not in tail and "runtime error:" not in tail, tail
