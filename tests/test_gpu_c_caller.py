"""The C ABI driven on the GPU from a plain C program (tests/c_gpu_caller.c):
HIP runtime calls for memory and a stream, libhprms.so for the op, no torch
and no Python between them; the program checks every result against the CPU
oracle itself (residuals and the streamer bit-exact, outputs within 1 ulp).
It is built with the libraries (__graft_entry__.build(), tests/Makefile) and
run here as a child process."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_gpu_caller")


def test_plain_c_program_on_the_gpu():
    assert os.path.exists(EXE), "tests/c_gpu_caller is not built: run __graft_entry__.build()"
    print("running", EXE, flush=True)
    p = subprocess.run([EXE], capture_output=True, text=True, timeout=240)
    print(p.stdout, flush=True)
    assert p.returncode == 0 and p.stdout.strip().endswith("ok"), p.stdout[-4000:] + p.stderr[-2000:]
    assert p.stdout.count("case ") == 8 and "FAIL" not in p.stdout
