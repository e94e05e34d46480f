"""The C ABI from C (tests/c_abi/nuq_check.c): dequant, GEMV, M=8 GEMM,
top-k, argmax and refusals through include/*.h with raw device pointers, no
Python in the loop, each checked against the oracle's C functions. Built by
__graft_entry__.build() (tests/c_abi/Makefile)."""
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent / "c_abi" / "_build" / "nuq_check"


def test_c_abi_from_c():
    assert EXE.exists(), f"{EXE} is missing: run __graft_entry__.build()"
    r = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    assert r.returncode == 0 and "nuq_check: OK" in r.stdout, r.stdout + r.stderr
