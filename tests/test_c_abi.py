"""The C ABI driven from plain C (tests/c_abi/abi_check.c, built by make with
the library): append, decode against a double-precision host computation,
the allocation-free entry point and the error path, with no Python or torch
in the calling process. Run as a child process."""

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(ROOT, "tests", "c_abi", "abi_check")


def test_abi_check_is_built():
    assert os.access(BINARY, os.X_OK), "tests/c_abi/abi_check is not built (run make)"


@pytest.mark.gpu
def test_c_caller_of_the_abi(gpu):
    print("c_abi: running tests/c_abi/abi_check", flush=True)
    done = subprocess.run([BINARY], capture_output=True, text=True, timeout=120)
    print(done.stdout, flush=True)
    assert done.returncode == 0, done.stdout + done.stderr
    assert "abi_check: OK" in done.stdout
