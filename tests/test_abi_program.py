"""The C ABI from a C++ host program (tests/abi_host_program.cpp, built by
__graft_entry__.build() against include/prism.h and libprism.so): layout,
synthetic blob, validation, fragment packing and the aux size on the host;
with a GPU, the reference's per-block stage sequence (attn -> router ->
experts) against the captured chain, bit for bit."""
import os
import subprocess

import pytest

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "abi_host_program.bin")


def run(*args):
    if not os.path.exists(EXE):
        pytest.fail(f"{EXE} is missing: run __graft_entry__.build()")
    r = subprocess.run([EXE, *args], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stderr
    assert r.stdout.startswith("ABI OK")
    return r.stdout


def test_abi_program_host_side():
    run()


@pytest.mark.gpu
def test_abi_program_stage_sequence_equals_chain():
    out = run("gpu")
    assert "stage calls == chain" in out
